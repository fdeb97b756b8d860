// Fused bf16 q/k/v kernels of the causal RACE layer, specialised for the hot path
// (compile-time bucket tile ST, head dim DP, hash bits KB; sub-chunk C = 32 tokens).
//
// Same math and block decomposition as race_scan_kernels.h (see race_scan.h), with
// the data flow arranged so that every MFMA accumulator is produced in the layout
// its consumer needs:
//  * the projection is computed transposed, acc[j][t] with j = table*4 + bit, so
//    one lane holds all K soft bits of one (token, table) pair and expands its 2^K
//    probabilities in registers (no LDS round trip of the projections);
//  * A is scanned transposed, A^T[s][t], so W = pQ / (A + eps) is written as
//    4-bucket vectors of one token row;
//  * the readout is accumulated transposed, out^T[d][t], and staged through LDS
//    for 16-byte coalesced global stores;
//  * the next sub-chunk's k, q, v (and go) rows are loaded into registers while the
//    current one is computed (two sub-chunks ahead in the forward totals);
//  * barrier phases per sub-chunk: 2 (forward totals), 4 (readout, backward totals),
//    5 (backward main, whose sub-chunk tail is pipelined into the next head).
#pragma once
#include <type_traits>

#include "race_scan.h"

namespace race {

RACE_DEV void zero_lds_bf16(__bf16 *p, int n, int tid, int nth)
{
    for (int i = tid; i < n; i += nth)
        p[i] = (__bf16)0.0f;
}

// Soft-hash of one table from its projections x[0..4) (rows >= KB are unused), in the exp2
// domain of the hardware exponential:
//   th_k = tanh(x_k),  u_k = th_k / scale,  a_k = exp(-2 u_k) = 2^(th_k * coef),
//   coef = -2 log2(e) / scale,
//   p[r] = prod_k sigmoid(2 c_k(r) u_k) = prod_{k: bit k of r clear} a_k / prod_k (1 + a_k),
// since sigmoid(2u) = 1 / (1 + a) and sigmoid(-2u) = a / (1 + a): one reciprocal per table.
// Bit k = 0 is the most significant bit of r (corner order of itertools.product([-1, 1])).
// The exponent is clamped to |u| <= 10: sigmoid(20) differs from 1 by 2e-9 (below fp32
// resolution next to 1) and den <= (1 + e^20)^4 < 2^117 stays finite at any temperature.
// mask = 0 gives all-zero probabilities (padding tokens and tables).
constexpr float SH_LOG2E = 1.4426950408889634f;
constexpr float SH_CLAMP = 20.0f * SH_LOG2E;

RACE_DEV float tanh_exp2(float x)
{
    return 1.0f - 2.0f * frcp(__builtin_amdgcn_exp2f(x * (2.0f * SH_LOG2E)) + 1.0f);
}

template <int KB>
RACE_DEV void probs_from_th(const float *th, float coef, float mask, float *p)
{
    float a[KB], den = 1.0f;
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        a[k] = __builtin_amdgcn_exp2f(__builtin_amdgcn_fmed3f(th[k] * coef, -SH_CLAMP, SH_CLAMP));
        den *= 1.0f + a[k];
    }
    p[0] = frcp(den) * mask;
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        const int n = 1 << k;
#pragma unroll
        for (int i = n - 1; i >= 0; --i) {
            const float pi = p[i];
            p[2 * i + 1] = pi;
            p[2 * i] = pi * a[k];
        }
    }
}

// th[0..4) = tanh of the projections (zero beyond KB) and the table's probabilities
template <int KB>
RACE_DEV void softhash_fwd_ct(const f32x4 &x, float coef, bool ok, float *th, float *p)
{
#pragma unroll
    for (int e = 0; e < 4; ++e)
        th[e] = e < KB ? tanh_exp2(x[e]) : 0.0f;
    probs_from_th<KB>(th, coef, ok ? 1.0f : 0.0f, p);
}

template <int ST, int DP, int KB, int NW>
struct FCfg {
    static constexpr int C = 32;
    static constexpr int NTH = NW * 64;
    // readout waves per SIMD asked of the register allocator: three workgroups of four waves
    // fit a CU's LDS at the bf16-output tile set of the 128-bucket, 64-dim variant
    static constexpr int RO_WAVES = (ST == 128 && DP == 64 && NW == 4 && KB >= 3) ? 3 : 1;
    static constexpr int R = 1 << KB;
    static constexpr int LT = ST / R;          // tables per bucket tile
    static constexpr int LTP = ((LT + 3) / 4) * 4;  // tables padded to whole projection tiles
    static constexpr int LKP = 4 * LTP;        // projection rows (4 per table, bits >= KB zero)
    static constexpr int NJT = LKP / 16;       // projection row tiles
    static constexpr int MTC = C / 16;         // token tiles
    static constexpr int NTS = ST / 16;
    static constexpr int NTD = DP / 16;
    static constexpr int NPT = NJT * MTC;      // projection tiles per tensor
    static constexpr int LDX = DP + 8;         // bf16 rows of tokens
    // k and q rows, read only as projection operands (16-byte MFMA reads of 16 rows): unpadded,
    // with the 16-byte chunks of row r stored at chunk ^ (r mod QCH) (kq_off), so both the row
    // stores (QCH threads per row) and the operand reads hit every bank once per pass (a pitch of
    // DP + 16 kept the reads conflict-free but made the stores conflict three ways)
    static constexpr int LDQ = DP;
    static constexpr int QCH = DP / 8;         // 16-byte chunks per k / q row
    static constexpr int LDC = C + 8;          // bf16 rows of length C
    static constexpr int LDS = ST + 8;         // bf16 rows of length ST
    static constexpr int LDG = ((LKP + 31) / 32) * 32 + 8;  // rows of projection grads (whole MFMA k steps)
    static constexpr int CHUNKS = C * DP / 8;  // 16-byte chunks of one token tile
    static constexpr int PF = (CHUNKS + NTH - 1) / NTH;
    static_assert(KB >= 2 && KB <= 4, "fused kernels: 2 <= K <= 4");
    static_assert(ST % R == 0 && ST % 32 == 0 && DP % 32 == 0, "tile shapes");
};

// Element offset of 16-byte chunk ch of row `row` in a k / q row tile (chunks XOR-swizzled by row).
template <class CF>
RACE_DEV int kq_off(int row, int ch)
{
    static_assert((CF::QCH & (CF::QCH - 1)) == 0, "power-of-two chunks per k / q row");
    return row * CF::LDQ + 8 * (ch ^ (row & (CF::QCH - 1)));
}

// Lane-constant operand fragments (loaded once per workgroup). Projection tiles
// are assigned to waves as t = wave + i*NW over NT tiles (k tiles, then q tiles);
// slot i holds the planes fragment of tile t's projection rows.
template <class CF, int DP, int NSLOT>
struct FusedFrags {
    bf16x8 proj[NSLOT][DP / 32];  // A operand: rows j = table*4 + bit, k = d
    bf16x8 tri[CF::MTC];          // B operand of the A scan: col t, k = tau, (tau <= t)

    RACE_DEV void load(const ScanParams &P, int l0, int Lt_valid, int lane, int wave)
    {
        const int LKtot = P.L * P.K;
#pragma unroll
        for (int i = 0; i < NSLOT; ++i) {
            const int t = wave + i * (CF::NTH / 64);
            const int jt = (t % CF::NPT) / CF::MTC;
            const int j = jt * 16 + (lane & 15);
            const int table = j >> 2, bit = j & 3;
#pragma unroll
            for (int kb = 0; kb < DP / 32; ++kb) {
                bf16x8 f;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int d = kb * 32 + (lane >> 4) * 8 + e;
                    float x = 0.0f;
                    if (bit < P.K && table < Lt_valid && d < P.D)
                        x = P.planes[d * LKtot + (l0 + table) * P.K + bit];
                    f[e] = (__bf16)x;
                }
                proj[i][kb] = f;
            }
        }
#pragma unroll
        for (int tt = 0; tt < CF::MTC; ++tt) {
            const int t = tt * 16 + (lane & 15);
            bf16x8 f;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                f[e] = (__bf16)(((lane >> 4) * 8 + e <= t) ? 1.0f : 0.0f);
            tri[tt] = f;
        }
    }

    RACE_DEV bf16x8 tri_of(int tt) const
    {
        bf16x8 r = tri[0];
#pragma unroll
        for (int i = 1; i < CF::MTC; ++i)
            if (tt == i)
                r = tri[i];
        return r;
    }
};

// acc[j][t] for the projection tile in slot i (rows j from registers), B = x rows t.
template <class CF, int DP, int NSLOT>
RACE_DEV f32x4 proj_T(const FusedFrags<CF, DP, NSLOT> &fr, int i, const __bf16 *sX, int tt, int lane)
{
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const int row = tt * 16 + (lane & 15);
#pragma unroll
    for (int kb = 0; kb < DP / 32; ++kb)
        EngBF16::mma(acc, fr.proj[i][kb], *reinterpret_cast<const bf16x8 *>(sX + kq_off<CF>(row, kb * 4 + (lane >> 4))));
    return acc;
}

// acc += A[m0.., k] B[n0.., k]^T over K (bf16 LDS operands, k-contiguous rows)
template <int K, int LDA, int LDB>
RACE_DEV void mma_ab(f32x4 &acc, const __bf16 *A, int m0, const __bf16 *B, int n0, int lane)
{
    const __bf16 *pa = A + (m0 + (lane & 15)) * LDA + (lane >> 4) * 8;
    const __bf16 *pb = B + (n0 + (lane & 15)) * LDB + (lane >> 4) * 8;
#pragma unroll
    for (int k = 0; k < K; k += 32)
        EngBF16::mma(acc, *reinterpret_cast<const bf16x8 *>(pa + k), *reinterpret_cast<const bf16x8 *>(pb + k));
}

// two fp32 values rounded to bf16 (round to nearest even) and packed into one dword, a in the low
// half: one v_cvt_pk_bf16_f32 (element-wise casts of a whole vector sometimes lower to two
// single conversions and a byte permute instead)
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
RACE_DEV uint32_t pk_bf16(float a, float b)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// store 4 accumulator rows (m0 + 4g + e) of column n as one vector: buf[n][m0+4g .. +3]
RACE_DEV void st_vec4(__bf16 *p, const f32x4 &v)
{
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u32x2 *>(p) = u32x2{pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3])};
}

// Operand pairs for MFMA chains whose reduction index k is a bucket or head-dim index held
// by accumulator tiles: the reduction order of an MFMA is free, so lane group g may supply
// k = k0 + 4g .. +3 and k0 + 16 + 4g .. +3 (the rows of two 16-row accumulator tiles) as
// its 8 consecutive k, as long as both operands use the same order.
// A operand from two accumulator tiles (rows k, col m = lane%16), converted to bf16.
RACE_DEV bf16x8 acc_pair(const f32x4 &lo, const f32x4 &hi)
{
    const u32x4 u = {pk_bf16(lo[0], lo[1]), pk_bf16(lo[2], lo[3]), pk_bf16(hi[0], hi[1]), pk_bf16(hi[2], hi[3])};
    return __builtin_bit_cast(bf16x8, u);
}

// The matching operand from an LDS array stored [n][k] (k contiguous): row n0 + lane%16.
RACE_DEV bf16x8 ld_pair(const __bf16 *X, int ld, int n0, int k0, int lane)
{
    const __bf16 *p = X + (n0 + (lane & 15)) * ld + k0 + 4 * (lane >> 4);
    const bf16x4 a = *reinterpret_cast<const bf16x4 *>(p);
    const bf16x4 b = *reinterpret_cast<const bf16x4 *>(p + 16);
    bf16x8 f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        f[e] = a[e];
        f[4 + e] = b[e];
    }
    return f;
}

// MFMA operand fragment (row m0 + lane%16, k = k0 + 8*(lane/16) .. +7) from an LDS array
// stored [m][k] (k contiguous): one 16-byte read.
RACE_DEV bf16x8 ld_k(const __bf16 *X, int ld, int m0, int k0, int lane)
{
    return *reinterpret_cast<const bf16x8 *>(X + (m0 + (lane & 15)) * ld + k0 + (lane >> 4) * 8);
}

// The same fragment from an LDS array stored [k][m] (m contiguous), with two transposing
// 64-bit reads (ds_read_b64_tr_b16). Within each 16-lane group, lane i receives element
// i % 4 of the 8-byte rows read by lanes i/4 + 4e (e = 0..3); so lane s of group g reads
// row k0 + 8g + s/4 (+4 for the second read) at columns m0 + 4*(s%4) .. +3, and lane i
// ends up holding column m0 + i of rows k0 + 8g .. k0 + 8g + 7.
RACE_DEV bf16x8 ld_tr(const __bf16 *X, int ld, int k0, int m0, int lane)
{
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    const int s = lane & 15;
    const __bf16 *p = X + (k0 + 8 * (lane >> 4) + (s >> 2)) * ld + m0 + 4 * (s & 3);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(p));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(p + 4 * ld));
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x8 r = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8, r);
}

// 16-byte chunk loads of one C x DP bf16 token tile (rows t0.., nv >= 1 valid rows). Rows at
// and beyond nv re-read row nv - 1 and are zeroed when stored: the destination registers are
// never written before the load, so issuing the next tile's loads needs no wait on earlier
// memory operations.
template <class CF>
RACE_DEV void tile_load(u32x4 (&r)[CF::PF], const __bf16 *base, int64_t st, int nv, int tid)
{
    constexpr int CH = CF::CHUNKS / CF::C;  // chunks per row
#pragma unroll
    for (int i = 0; i < CF::PF; ++i) {
        const int idx = tid + i * CF::NTH;
        const int row = min(idx / CH, nv - 1), c = idx % CH;
        // (no branch when every thread loads whole chunk sets: a fixed number of loads per
        // thread lets in-order memory-counter waits skip the newest loads)
        if (CF::CHUNKS % CF::NTH == 0 || idx < CF::CHUNKS)
            r[i] = *reinterpret_cast<const u32x4 *>(base + row * (int)st + c * 8);
    }
}

// k or q tile rows into LDS in the swizzled layout of kq_off (rows at and beyond nv as loaded).
template <class CF>
RACE_DEV void tile_store_kq(__bf16 *dst, const u32x4 (&r)[CF::PF], int tid)
{
    constexpr int CH = CF::CHUNKS / CF::C;
    static_assert(CH == CF::QCH, "one k / q row per QCH chunks");
#pragma unroll
    for (int i = 0; i < CF::PF; ++i) {
        const int idx = tid + i * CF::NTH;
        if (idx < CF::CHUNKS)
            *reinterpret_cast<u32x4 *>(dst + kq_off<CF>(idx / CH, idx % CH)) = r[i];
    }
}

// Tile rows into LDS, rows at and beyond nv as loaded (copies of row nv - 1) or, with ZERO, as
// zeros. The copies are finite, and every product the fused kernels form with a padding token's
// row is multiplied by that token's zero probabilities (pK, pQ and so W are masked to zero by the
// soft-hash), or lands in an output row that is not stored: no kernel needs the zeros.
template <class CF, bool ZERO = false, int LD = CF::LDX>
RACE_DEV void tile_store_rows(__bf16 *dst, const u32x4 (&r)[CF::PF], int nv, int tid)
{
    constexpr int CH = CF::CHUNKS / CF::C;
#pragma unroll
    for (int i = 0; i < CF::PF; ++i) {
        const int idx = tid + i * CF::NTH;
        if (idx < CF::CHUNKS) {
            const bool ok = !ZERO || idx / CH < nv;
            const u32x4 x = {ok ? r[i][0] : 0u, ok ? r[i][1] : 0u, ok ? r[i][2] : 0u, ok ? r[i][3] : 0u};
            *reinterpret_cast<u32x4 *>(dst + (idx / CH) * LD + (idx % CH) * 8) = x;
        }
    }
}

// Inclusive prefix sum over the 16 lanes of each DPP row (Hillis-Steele with row_shr and zero
// fill: four VALU adds, no LDS).
RACE_DEV float row_scan16(float v)
{
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x111, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x112, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x114, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x118, 0xF, 0xF, true));
    return v;
}

// Value of lane 15 of each 16-lane DPP row, in every lane of that row (row_newbcast:15).
RACE_DEV float row_bcast15(float v)
{
    // every lane has a source lane: no old value to keep (and no zero move ahead of the DPP move)
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x15F, 0xF, 0xF, false));
}

// s_waitcnt vmcnt(0): every vector-memory operation of the wave has completed. Issued once
// after a kernel's prologue loads, so that the uses of those registers inside the sub-chunk
// loop need no wait there (such a wait would also cover the loop's own prefetch loads).
RACE_DEV void wait_vmem_all()
{
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt 0, expcnt 7 (none), lgkmcnt 15 (none)
}

// s_waitcnt vmcnt(N): all but the N most recently issued vector-memory operations have completed
template <int N>
RACE_DEV void wait_vmem_older()
{
    static_assert(N >= 0 && N < 16, "vmcnt immediate (low field)");
    __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

RACE_DEV const __bf16 *row_ptr(const View &v, int b, int h, int t)
{
    return reinterpret_cast<const __bf16 *>(v.p) + (b * v.sb + h * v.sh + (int64_t)t * v.st);
}

// Bucket tiles launched one after another (OutView::stage_f32): each thread owns E consecutive
// elements of one row of a staged C x DP output tile. The earlier tiles' fp32 sum for those
// elements (OutView::acc) is loaded into registers some barrier phases before the tile is stored,
// so that the store does not wait on HBM; zeros when there is no earlier tile.
template <int C, int DP, int NTH>
struct AccRows {
    static constexpr int E = C * DP / NTH;  // elements per thread
    static constexpr int RPT = DP / E;      // threads per row
    static_assert(E % 4 == 0 && E <= 16 && RPT * E == DP, "accumulated store layout");
    f32x4 a[E / 4];

    RACE_DEV void load(const OutView &o, int b, int h, int t0, int nv, int tid)
    {
        const int row = tid / RPT, col = (tid % RPT) * E;
#pragma unroll
        for (int i = 0; i < E / 4; ++i)
            a[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (o.acc && row < nv) {
            const float *p = o.acc + b * o.acc_sb + h * o.acc_sh + (int64_t)(t0 + row) * o.acc_st + col;
#pragma unroll
            for (int i = 0; i < E / 4; ++i)
                a[i] = *reinterpret_cast<const f32x4 *>(p + 4 * i);
        }
    }
};

// Store of an fp32-staged tile in that mode: staged values plus the loaded earlier-tile sum, as
// fp32 (the running sum, or an fp32 output) or rounded once to bf16 (the last tile).
template <int C, int DP, int LDO, int NTH>
RACE_DEV void store_staged_acc(const OutView &o, int b, int h, int st, int t0, int nv, const float (*sO)[LDO],
                               const AccRows<C, DP, NTH> &ar, int tid)
{
    using AR = AccRows<C, DP, NTH>;
    constexpr int E = AR::E;
    const int row = tid / AR::RPT, col = (tid % AR::RPT) * E;
    if (row >= nv)
        return;
    f32x4 x[E / 4];
#pragma unroll
    for (int i = 0; i < E / 4; ++i)
        x[i] = *reinterpret_cast<const f32x4 *>(&sO[row][col + 4 * i]) + ar.a[i];
    const int64_t off = (int64_t)st * o.tile + b * o.sb + h * o.sh + (int64_t)(t0 + row) * o.st + col;
    if (o.f32) {
        float *dst = reinterpret_cast<float *>(o.p) + off;
#pragma unroll
        for (int i = 0; i < E / 4; ++i)
            *reinterpret_cast<f32x4 *>(dst + 4 * i) = x[i];
    } else if constexpr (E == 4) {
        bf16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w[e] = (__bf16)x[0][e];
        *reinterpret_cast<bf16x4 *>(reinterpret_cast<__bf16 *>(o.p) + off) = w;
    } else {
#pragma unroll
        for (int i = 0; i < E / 8; ++i) {
            bf16x8 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                w[e] = (__bf16)x[2 * i][e];
                w[4 + e] = (__bf16)x[2 * i + 1][e];
            }
            *reinterpret_cast<bf16x8 *>(reinterpret_cast<__bf16 *>(o.p) + off + 8 * i) = w;
        }
    }
}

// Coalesced store of a staged C x DP tile (rows < nv) to a [B][H][T][D] output view.
template <class OT, int C, int DP, int LDO, int NTH>
RACE_DEV void store_staged(const OutView &o, int b, int h, int st, int t0, int nv, const OT (*sO)[LDO], int tid)
{
    constexpr int EPC = 16 / (int)sizeof(OT);  // elements per 16-byte chunk
    constexpr int OCH = DP / EPC;
    for (int i = tid; i < C * OCH; i += NTH) {
        const int row = i / OCH, ch = i % OCH;
        if (row < nv) {
            OT *dst = reinterpret_cast<OT *>(o.p) + (int64_t)st * o.tile + b * o.sb + h * o.sh +
                      (int64_t)(t0 + row) * o.st + ch * EPC;
            *reinterpret_cast<u32x4 *>(dst) = *reinterpret_cast<const u32x4 *>(&sO[row][ch * EPC]);
        }
    }
}

// Store of a staged output tile: the accumulating form when the bucket tiles run one launch
// after another (fp32 staging only), the plain one otherwise.
template <class OT, int C, int DP, int LDO, int NTH>
RACE_DEV void store_out(const OutView &o, int b, int h, int st, int t0, int nv, const OT (*sO)[LDO],
                        const AccRows<C, DP, NTH> &ar, int tid)
{
    if constexpr (std::is_same<OT, float>::value) {
        if (o.stage_f32) {  // uniform branch
            store_staged_acc<C, DP, LDO, NTH>(o, b, h, st, t0, nv, sO, ar, tid);
            return;
        }
    }
    store_staged<OT, C, DP, LDO, NTH>(o, b, h, st, t0, nv, sO, tid);
}

// ============================================================================ forward totals
template <int ST, int DP, int KB, int NW>
__global__ __launch_bounds__(NW * 64) void race_fused_fwd_totals(const ScanParams P)
{
    using CF = FCfg<ST, DP, KB, NW>;
    constexpr int C = CF::C, NTH = CF::NTH, R = CF::R;
    __shared__ __align__(16) __bf16 sK[C][CF::LDQ];
    __shared__ __align__(16) __bf16 sV[2][C][CF::LDX];  // by sub-chunk parity
    __shared__ __align__(16) __bf16 sPK[C][CF::LDS];  // rows [t][s]

    const Ctx c = make_ctx(P, ST);
    const float coef = -2.0f * SH_LOG2E * P.inv_scale;  // soft-hash exponent factor
    const int tid = c.tid, lane = c.lane, wave = c.wave;
    __builtin_assume(wave >= 0 && wave < NW);  // (threadIdx.x < NW * 64): per-wave tile counts that divide evenly need no guard
    constexpr int TPW_S = (CF::NTS * CF::NTD + NW - 1) / NW;
    constexpr int TPW_A = (CF::NTS + NW - 1) / NW;
    constexpr int TPW_P = (CF::NPT + NW - 1) / NW;
    FusedFrags<CF, DP, TPW_P> fr;
    fr.load(P, c.l0, c.Lt, lane, wave);
    f32x4 accS[TPW_S], accA[TPW_A];
#pragma unroll
    for (int i = 0; i < TPW_S; ++i)
        accS[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < TPW_A; ++i)
        accA[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e)
        ones[e] = (__bf16)1.0f;

    const int nsub = (c.t_end - c.t_begin + C - 1) / C;
    // rows of sub-chunk sc + 1 are in flight while sub-chunk sc is computed and the loads of
    // sc + 2 are issued at its start (twice the bytes in flight of a one-step prefetch, which
    // bounded this kernel by latency): two register sets, the loop unrolled by two so that each
    // set is named statically. Every thread issues exactly 2 * PF loads per sub-chunk, so
    // "vmcnt <= 2 * PF" means that all but the newest set have landed.
    static_assert(CF::CHUNKS % CF::NTH == 0, "every thread loads whole chunk sets");
    u32x4 pkA[CF::PF], pvA[CF::PF], pkB[CF::PF], pvB[CF::PF];
    auto load_rows = [&](u32x4 (&rk)[CF::PF], u32x4 (&rv)[CF::PF], int t1) {
        tile_load<CF>(rk, row_ptr(P.k, c.b, c.hk, t1), P.k.st, min(C, c.t_end - t1), tid);
        tile_load<CF>(rv, row_ptr(P.v, c.b, c.hk, t1), P.v.st, min(C, c.t_end - t1), tid);
    };
    const int t_last = c.t_begin + (nsub - 1) * C;  // start of the last sub-chunk
    load_rows(pkB, pvB, c.t_begin);
    wait_vmem_all();
    tile_store_kq<CF>(&sK[0][0], pkB, tid);
    tile_store_rows<CF>(&sV[0][0][0], pvB, min(C, c.t_end - c.t_begin), tid);
    load_rows(pkA, pvA, min(c.t_begin + C, t_last));
    __syncthreads();

    // two barrier phases per sub-chunk: soft-hash of k, then the MFMAs together with the next
    // sub-chunk's rows into LDS (k rows are free once hashed, v rows double buffered)
    auto body = [&](int sc, u32x4 (&nk)[CF::PF], u32x4 (&nvr)[CF::PF], u32x4 (&fk)[CF::PF], u32x4 (&fv)[CF::PF]) {
        const int t0 = c.t_begin + sc * C;
        const int nv = min(C, c.t_end - t0);
        const int cur = sc & 1, nxt = cur ^ 1;
        // issued unconditionally (a straight-line load stream keeps the compiler's memory-counter
        // waits exact): past the end it re-reads the last sub-chunk, whose rows are not used
        load_rows(fk, fv, min(t0 + 2 * C, t_last));
        // soft-hash of k -> pK rows
#pragma unroll
        for (int i = 0; i < TPW_P; ++i) {
            const int t = wave + i * NW;
            if (t < CF::NPT) {
                const int jt = t / CF::MTC, tt = t % CF::MTC;
                const f32x4 acc = proj_T<CF, DP, TPW_P>(fr, i, &sK[0][0], tt, lane);
                const int tok = tt * 16 + (lane & 15), table = jt * 4 + (lane >> 4);
                const bool ok = tok < nv && table < c.Lt;
                float th[4], p[R];
                softhash_fwd_ct<KB>(acc, coef, ok, th, p);
                if (table < CF::LT) {
#pragma unroll
                    for (int h = 0; h < R / 4; ++h) {
                        bf16x4 w;
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            w[e] = (__bf16)p[4 * h + e];
                        *reinterpret_cast<bf16x4 *>(&sPK[tok][table * R + 4 * h]) = w;
                    }
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < TPW_S; ++i) {
            const int t = wave + i * NW;
            if (t < CF::NTS * CF::NTD)
                EngBF16::mma(accS[i], ld_tr(&sPK[0][0], CF::LDS, 0, (t / CF::NTD) * 16, lane),
                             ld_tr(&sV[cur][0][0], CF::LDX, 0, (t % CF::NTD) * 16, lane));
        }
#pragma unroll
        for (int i = 0; i < TPW_A; ++i) {
            const int tn = wave + i * NW;
            if (tn < CF::NTS)
                EngBF16::mma(accA[i], ones, ld_tr(&sPK[0][0], CF::LDS, 0, tn * 16, lane));
        }
        // the next rows go to LDS unconditionally (after the last sub-chunk they are zeros that
        // nothing reads): every prefetch set is consumed on every path, so the compiler's
        // memory-counter tracking needs no wait before the set is loaded again
        wait_vmem_older<2 * CF::PF>();
        tile_store_kq<CF>(&sK[0][0], nk, tid);
        tile_store_rows<CF>(&sV[nxt][0][0], nvr, min(C, c.t_end - t0 - C), tid);
        __syncthreads();
    };
    for (int sc = 0; sc < nsub; sc += 2) {
        body(sc, pkA, pvA, pkB, pvB);
        if (sc + 1 < nsub)
            body(sc + 1, pkB, pvB, pkA, pvA);
    }
    wait_vmem_all();

    const int64_t slot = (int64_t)c.z * (P.NB + 1) + c.blk;
    float *wB = P.wsB + (slot * P.S_pad + c.s0) * P.DPw;
#pragma unroll
    for (int i = 0; i < TPW_S; ++i) {
        const int t = wave + i * NW;
        if (t < CF::NTS * CF::NTD) {
            const int r = acc_row((t / CF::NTD) * 16, lane), col = acc_col((t % CF::NTD) * 16, lane);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                wB[(int64_t)(r + e) * P.DPw + col] = accS[i][e];
        }
    }
    float *wA = P.wsA + slot * P.S_pad + c.s0;
#pragma unroll
    for (int i = 0; i < TPW_A; ++i) {
        const int tn = wave + i * NW;
        if (tn < CF::NTS && lane < 16)
            wA[tn * 16 + lane] = accA[i][0];
    }
}

// Wave-uniform copy of a 64-bit integer (or address) that holds the same value in every lane (a
// per-wave choice between kernel arguments), so that the address arithmetic on it runs on the
// scalar unit.
RACE_DEV int64_t uniform_i64(int64_t x)
{
    const uint64_t v = (uint64_t)x;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Row loads of a group of four waves (the movers of the wave-specialised backward kernels, the
// forward readout's workgroup): one 16-byte chunk of each of two C x 64 bf16 token tiles per
// thread, from two [B][H][T][D] tensors (which may be a per-wave choice). Their block row-0
// pointers and row strides are made wave-uniform once, so a sub-chunk's row-0 address is scalar
// arithmetic and a thread's chunk is that address plus a 32-bit byte offset (the global_load form with a scalar base): a clamp and a 24-bit multiply-add
// per load instead of 64-bit address arithmetic on every lane. Rows at and beyond nv (the valid
// rows of the sub-chunk) re-read row nv - 1. Needs row strides below 2^24 elements (checked on
// the host), so row * stride + column stays below 2^29 elements and its byte offset in 32 bits.
struct MoverRows {
    typedef const __attribute__((address_space(1))) char gchar;  // global memory, byte addressed
    typedef const __attribute__((address_space(1))) u32x4 gu32x4;
    gchar *pa, *pb;
    int64_t sa, sb;  // row strides in bytes
    int row, col;    // the thread's row within the tile and element offset within the row

    // a / b: this wave's two tensors (a per-wave choice, made wave-uniform here, after the choice)
    RACE_DEV void init(const __bf16 *a, int64_t sta, const __bf16 *b, int64_t stb, int mid, int chunks_per_row)
    {
        pa = (gchar *)(uint64_t)uniform_i64((int64_t)reinterpret_cast<uintptr_t>(a));
        pb = (gchar *)(uint64_t)uniform_i64((int64_t)reinterpret_cast<uintptr_t>(b));
        sa = uniform_i64(sta) * 2;
        sb = uniform_i64(stb) * 2;
        row = mid / chunks_per_row;
        col = (mid % chunks_per_row) * 8;
    }

    // rows t_off .. t_off + C - 1 of the block (t_off = sub-chunk index * C)
    RACE_DEV void load(u32x4 &ra, u32x4 &rb, int t_off, int nv) const
    {
        const unsigned rr = (unsigned)min(row, nv - 1);
        const unsigned oa = (__umul24(rr, (unsigned)(sa >> 1)) + col) * 2u;
        const unsigned ob = (__umul24(rr, (unsigned)(sb >> 1)) + col) * 2u;
        ra = *reinterpret_cast<gu32x4 *>(pa + t_off * sa + (uint64_t)oa);
        rb = *reinterpret_cast<gu32x4 *>(pb + t_off * sb + (uint64_t)ob);
    }
    // the first tensor's chunk only
    RACE_DEV void load_a(u32x4 &ra, int t_off, int nv) const
    {
        const unsigned rr = (unsigned)min(row, nv - 1);
        const unsigned oa = (__umul24(rr, (unsigned)(sa >> 1)) + col) * 2u;
        ra = *reinterpret_cast<gu32x4 *>(pa + t_off * sa + (uint64_t)oa);
    }
};

// ============================================================================ forward readout
template <int ST, int DP, int KB, int NW, bool OUT_F32, bool G1>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(FCfg<ST, DP, KB, NW>::RO_WAVES)))
void race_fused_fwd_readout(const ScanParams P)
{
    using CF = FCfg<ST, DP, KB, NW>;
    constexpr int C = CF::C, NTH = CF::NTH, R = CF::R, MTC = CF::MTC;
    // pK rows at a pitch of ST + 16 elements: its 16-byte MFMA operand reads (the triu product) hit
    // every bank once per pass (two-way conflicts at ST + 8)
    constexpr int LDX = CF::LDX, LDC = CF::LDC, LDS = CF::LDS, LDK = CF::LDS + 8;
    using OT = typename std::conditional<OUT_F32, float, __bf16>::type;
    constexpr int LDO = DP + (OUT_F32 ? 4 : 8);
    __shared__ __align__(16) __bf16 sK[C][CF::LDQ];
    __shared__ __align__(16) __bf16 sQ[C][CF::LDQ];
    __shared__ __align__(16) __bf16 sV[2][C][LDX];   // v rows, double buffered
    __shared__ __align__(16) __bf16 sPK[C][LDK];     // rows [t][s]
    __shared__ __align__(16) __bf16 sPQ[C][LDS];
    __shared__ __align__(16) __bf16 sPm[C][LDC];
    // W (written in P2, read in P3) and the output staging (written in P4, read in the next
    // step's P1) share one buffer: barriers separate every use of one from the other
    constexpr int SZ_W = C * LDS * 2 > C * LDO * (int)sizeof(OT) ? C * LDS * 2 : C * LDO * (int)sizeof(OT);
    __shared__ __align__(16) char uW[SZ_W];
    __bf16(*sW)[LDS] = reinterpret_cast<__bf16(*)[LDS]>(uW);
    OT(*sO)[LDO] = reinterpret_cast<OT(*)[LDO]>(uW);
    __shared__ __align__(16) float sA0[2][ST];

    const Ctx c = make_ctx(P, ST);
    const float coef = -2.0f * SH_LOG2E * P.inv_scale;  // soft-hash exponent factor
    const int tid = c.tid, lane = c.lane, wave = c.wave;
    __builtin_assume(wave >= 0 && wave < NW);  // (threadIdx.x < NW * 64): per-wave tile counts that divide evenly need no guard
    constexpr int TPW_P0 = (2 * CF::NPT + NW - 1) / NW;
    FusedFrags<CF, DP, TPW_P0> fr;
    fr.load(P, c.l0, c.Lt, lane, wave);
    zero_lds_bf16(&sPK[0][0], C * LDK, tid, NTH);
    zero_lds_bf16(&sPQ[0][0], C * LDS, tid, NTH);

    constexpr int TPW_S = (CF::NTS * CF::NTD + NW - 1) / NW;  // state tiles [ST x DP]
    constexpr int TPW_A = (CF::NTS * MTC + NW - 1) / NW;      // A^T tiles [ST x C]
    // out^T tiles [DP x C]: wave w owns head-dim tiles w + NW*j (j < NDW) for both token
    // tiles, the same head-dim tiles as its state tiles accS, so out^T = St^T W^T takes its A
    // operand straight from the state accumulators
    static_assert(CF::NTD % NW == 0, "head-dim tiles must split evenly over the waves");
    constexpr int NDW = CF::NTD / NW;
    constexpr int TPW_O = NDW * MTC;
    constexpr int TPW_M = (MTC * MTC + NW - 1) / NW;          // Pm^T tiles [C x C]
    constexpr int NPT2 = 2 * CF::NPT;                         // k and q projection tiles
    constexpr int TPW_P = (NPT2 + NW - 1) / NW;

    const int64_t slot = (int64_t)c.z * (P.NB + 1) + c.blk;
    f32x4 accS[TPW_S];
    {
        const float *wB = P.wsB + (slot * P.S_pad + c.s0) * P.DPw;
#pragma unroll
        for (int i = 0; i < TPW_S; ++i) {
            const int t = wave + i * NW;
            accS[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (t < CF::NTS * CF::NTD) {
                const int m0 = (t / CF::NTD) * 16, n0 = (t % CF::NTD) * 16;
                const int r = acc_row(m0, lane), col = acc_col(n0, lane);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    accS[i][e] = wB[(int64_t)(r + e) * P.DPw + col];
            }
        }
        const float *wA = P.wsA + slot * P.S_pad + c.s0;
        for (int s = tid; s < ST; s += NTH)
            sA0[0][s] = wA[s] + P.eps;  // the carry holds A + eps
    }

    const int G = G1 ? 1 : P.G;  // G1: one query head per kv head, the head loop folds away
    const int nsub = (c.t_end - c.t_begin + C - 1) / C;
    u32x4 pk[CF::PF], pq[CF::PF], pv[CF::PF];
    // one 16-byte chunk per thread (D = 64 on four waves): the prefetch of the next rows forms its
    // addresses from wave-uniform block row-0 pointers plus a 32-bit lane offset (MoverRows)
    constexpr bool SB = CF::CHUNKS == NTH && DP == 64;
    MoverRows mvKV, mvQ;
    if constexpr (SB) {
        mvKV.init(row_ptr(P.k, c.b, c.hk, c.t_begin), P.k.st, row_ptr(P.v, c.b, c.hk, c.t_begin), P.v.st, tid, DP / 8);
        mvQ.init(row_ptr(P.q, c.b, c.hk * G, c.t_begin), P.q.st, row_ptr(P.q, c.b, c.hk * G, c.t_begin), P.q.st, tid,
                 DP / 8);
    }
    {
        const int nv0 = min(C, c.t_end - c.t_begin);
        tile_load<CF>(pk, row_ptr(P.k, c.b, c.hk, c.t_begin), P.k.st, nv0, tid);
        tile_load<CF>(pq, row_ptr(P.q, c.b, c.hk * G, c.t_begin), P.q.st, nv0, tid);
        tile_load<CF>(pv, row_ptr(P.v, c.b, c.hk, c.t_begin), P.v.st, nv0, tid);
        tile_store_kq<CF>(&sK[0][0], pk, tid);
        tile_store_kq<CF>(&sQ[0][0], pq, tid);
        tile_store_rows<CF>(&sV[0][0][0], pv, nv0, tid);
    }
    wait_vmem_all();
    __syncthreads();

    f32x4 accA[TPW_A];  // 1/(A+eps), transposed tiles, kept across query heads
    int prev_t0 = -1, prev_nv = 0, prev_h = 0;
    AccRows<C, DP, NTH> arO;
    for (int sc = 0; sc < nsub; ++sc) {
        const int t0 = c.t_begin + sc * C;
        const int nv = min(C, c.t_end - t0);
        const int cur = sc & 1, nxt = cur ^ 1;
        const bool more = sc + 1 < nsub;
        if (more) {
            const int t1 = t0 + C, nv1 = min(C, c.t_end - t1);
            if constexpr (SB) {
                mvKV.load(pk[0], pv[0], t1 - c.t_begin, nv1);
                if (G == 1)
                    mvQ.load_a(pq[0], t1 - c.t_begin, nv1);
            } else {
                tile_load<CF>(pk, row_ptr(P.k, c.b, c.hk, t1), P.k.st, nv1, tid);
                tile_load<CF>(pv, row_ptr(P.v, c.b, c.hk, t1), P.v.st, nv1, tid);
                if (G == 1)
                    tile_load<CF>(pq, row_ptr(P.q, c.b, c.hk, t1), P.q.st, nv1, tid);
            }
        }
        for (int g = 0; g < G; ++g) {
            const int hq = c.hk * G + g;
            if (g > 0) {  // further query heads of the group: load q synchronously
                u32x4 tq[CF::PF];
                tile_load<CF>(tq, row_ptr(P.q, c.b, hq, t0), P.q.st, nv, tid);
                tile_store_kq<CF>(&sQ[0][0], tq, tid);
                __syncthreads();
            }
            // ---- P1: soft-hash of k (first head only) and q; previous output rows to HBM
#pragma unroll
            for (int i = 0; i < TPW_P; ++i) {
                const int t = wave + i * NW;
                const bool isk = t < CF::NPT;
                if (t < NPT2 && (isk ? g == 0 : true)) {
                    const int tq_ = isk ? t : t - CF::NPT;
                    const int jt = tq_ / MTC, tt = tq_ % MTC;
                    const f32x4 acc = proj_T<CF, DP, TPW_P0>(fr, i, isk ? &sK[0][0] : &sQ[0][0], tt, lane);
                    const int tok = tt * 16 + (lane & 15), table = jt * 4 + (lane >> 4);
                    const bool ok = tok < nv && table < c.Lt;
                    float th[4], p[R];
                    softhash_fwd_ct<KB>(acc, coef, ok, th, p);
                    bf16x8 v8[R / 8 > 0 ? R / 8 : 1];
                    bf16x4 v4;
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const __bf16 x = (__bf16)p[r];
                        if (R >= 8)
                            v8[r / 8][r % 8] = x;
                        else
                            v4[r] = x;
                    }
                    __bf16 *row = isk ? &sPK[tok][table * R] : &sPQ[tok][table * R];
                    if (table < CF::LT) {
                        if (R >= 8) {
#pragma unroll
                            for (int h = 0; h < R / 8; ++h)
                                *reinterpret_cast<bf16x8 *>(row + 8 * h) = v8[h];
                        } else {
                            *reinterpret_cast<bf16x4 *>(row) = v4;
                        }
                    }
                }
            }
            if (prev_t0 >= 0)  // coalesced store of the previous (sub-chunk, head) output from sO
                store_out<OT, C, DP, LDO, NTH>(P.out, c.b, prev_h, c.st, prev_t0, prev_nv, sO, arO, tid);
            __syncthreads();
            // ---- P2: A^T = A0 + pK^T Tri^T (first head); W^T = pQ^T / (A + eps) -> sW
            //          | (tiles one launch after another) the earlier tiles' sum of this step's
            //          output rows into registers, for the store in the next step's P1
            if constexpr (OUT_F32) {
                if (P.out.stage_f32)
                    arO.load(P.out, c.b, hq, t0, nv, tid);
            }
#pragma unroll
            for (int i = 0; i < TPW_A; ++i) {
                const int t = wave + i * NW;
                if (t < CF::NTS * MTC) {
                    const int ts = t / MTC, tt = t % MTC;
                    const int s = ts * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
                    if (g == 0) {
                        f32x4 a = *reinterpret_cast<const f32x4 *>(&sA0[cur][s]);
                        EngBF16::mma(a, ld_tr(&sPK[0][0], LDK, 0, ts * 16, lane), fr.tri_of(tt));
                        if (tt == MTC - 1 && (lane & 15) == 15)
                            *reinterpret_cast<f32x4 *>(&sA0[nxt][s]) = a;
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            accA[i][e] = frcp(a[e]);
                    }
                    const bf16x4 q4 = *reinterpret_cast<const bf16x4 *>(&sPQ[tok][s]);
                    f32x4 w;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        w[e] = (float)q4[e] * accA[i][e];
                    st_vec4(&sW[tok][s], w);
                }
            }
            __syncthreads();
            // ---- P3: Pm^T = triu-masked pK W^T -> sPm (first: its LDS stores then drain behind the
            //          products, 1.5 % faster) ; out^T = St^T W^T (state operand from registers) ;
            //          St += pK^T V (last head)
#pragma unroll
            for (int i = 0; i < TPW_M; ++i) {
                const int t = wave + i * NW;
                if (t < MTC * MTC) {
                    const int tu = t / MTC, tt = t % MTC;  // rows tau, cols t
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    mma_ab<ST, LDK, LDS>(acc, &sPK[0][0], tu * 16, &sW[0][0], tt * 16, lane);
                    const int tau = tu * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (tau + e > tok)
                            acc[e] = 0.0f;
                    st_vec4(&sPm[tok][tau], acc);
                }
            }
            f32x4 accO[TPW_O];
#pragma unroll
            for (int i = 0; i < TPW_O; ++i) {
                const int j = i / MTC, tt = i % MTC;
                accO[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < ST / 32; ++ks)
                    EngBF16::mma(accO[i], acc_pair(accS[(2 * ks) * NDW + j], accS[(2 * ks + 1) * NDW + j]),
                                 ld_pair(&sW[0][0], LDS, tt * 16, 32 * ks, lane));
            }
            if (g == G - 1) {
#pragma unroll
                for (int i = 0; i < TPW_S; ++i) {
                    const int t = wave + i * NW;
                    if (t < CF::NTS * CF::NTD)
                        EngBF16::mma(accS[i], ld_tr(&sPK[0][0], LDK, 0, (t / CF::NTD) * 16, lane),
                                     ld_tr(&sV[cur][0][0], LDX, 0, (t % CF::NTD) * 16, lane));
                }
            }
            __syncthreads();
            // ---- P4: out^T += V^T Pm^T -> sO ; next rows -> LDS
#pragma unroll
            for (int i = 0; i < TPW_O; ++i) {
                const int td = wave + NW * (i / MTC), tt = i % MTC;
                EngBF16::mma(accO[i], ld_tr(&sV[cur][0][0], LDX, 0, td * 16, lane),
                             ld_k(&sPm[0][0], LDC, tt * 16, 0, lane));
                const int d = td * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
                if constexpr (OUT_F32)
                    *reinterpret_cast<f32x4 *>(&sO[tok][d]) = accO[i];
                else
                    st_vec4(&sO[tok][d], accO[i]);
            }
            prev_t0 = t0;
            prev_nv = nv;
            prev_h = hq;
            wait_vmem_all();
            if (g == G - 1) {
                if (more) {
                    const int nv1 = min(C, c.t_end - t0 - C);
                    tile_store_kq<CF>(&sK[0][0], pk, tid);
                    tile_store_rows<CF>(&sV[nxt][0][0], pv, nv1, tid);
                    if (G == 1)
                        tile_store_kq<CF>(&sQ[0][0], pq, tid);
                    else {
                        u32x4 tq[CF::PF];
                        tile_load<CF>(tq, row_ptr(P.q, c.b, c.hk * G, t0 + C), P.q.st, nv1, tid);
                        tile_store_kq<CF>(&sQ[0][0], tq, tid);
                    }
                }
            }
            __syncthreads();
        }
    }
    // last output rows
    store_out<OT, C, DP, LDO, NTH>(P.out, c.b, prev_h, c.st, prev_t0, prev_nv, sO, arO, tid);
}


// Planes fragments for the soft-hash backward, dx^T = P gproj^T: A operand rows d of
// one 16-row head-dim tile, k = projection rows j (natural order, zero-padded bits).
template <class CF, int DP, int NSLOT>
struct BackFrags {
    bf16x8 f[NSLOT][CF::LKP / 32 > 0 ? CF::LKP / 32 : 1];

    RACE_DEV void load(const ScanParams &P, int l0, int Lt_valid, int lane, int wave, int ntiles_t)
    {
        const int LKtot = P.L * P.K;
#pragma unroll
        for (int i = 0; i < NSLOT; ++i) {
            const int t = wave + i * (CF::NTH / 64);
            const int td = t / ntiles_t;
            const int d = td * 16 + (lane & 15);
#pragma unroll
            for (int kb = 0; kb < (CF::LKP + 31) / 32; ++kb) {
                bf16x8 v;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int j = kb * 32 + (lane >> 4) * 8 + e;
                    const int table = j >> 2, bit = j & 3;
                    float x = 0.0f;
                    if (j < CF::LKP && bit < P.K && table < Lt_valid && d < P.D)
                        x = P.planes[d * LKtot + (l0 + table) * P.K + bit];
                    v[e] = (__bf16)x;
                }
                f[i][kb] = v;
            }
        }
    }
};

// Soft-hash backward of one (token, table): gproj[k] = dL/dproj_k from the table's
// probabilities p, its soft bits u and dL/dp (softmax + corner + tanh chain).
template <int KB>
RACE_DEV void softhash_bwd_ct(const float *th, const float *p, const float *gp, float inv_scale, float *gproj)
{
    constexpr int R = 1 << KB;
    float dot = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r)
        dot += p[r] * gp[r];
    // gz_r = dL/dz_r (softmax backward); gu_k = sum_r sign_k(r) gz_r, sign +1 where bit k of r
    // is set: a butterfly over the bits from the least significant one, pair sums feed the
    // next level and pair differences sum to that bit's gu
    float z[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
        z[r] = p[r] * (gp[r] - dot);
#pragma unroll
    for (int lvl = 0; lvl < KB; ++lvl) {
        const int k = KB - 1 - lvl;  // bit k of r is the lowest remaining index bit
        const int n = R >> (lvl + 1);
        float gu = 0.0f;
#pragma unroll
        for (int i = 0; i < n; ++i) {
            gu += z[2 * i + 1] - z[2 * i];
            z[i] = z[2 * i] + z[2 * i + 1];
        }
        gproj[k] = gu * inv_scale * (1.0f - th[k] * th[k]);
    }
}

// Register buffer for the k, v, q, go rows of the next (sub-chunk, head) step: loads are
// issued one step ahead and land in LDS at the start of the step that uses them.
template <class CF>
struct RowPrefetch {
    u32x4 k[CF::PF], v[CF::PF], q[CF::PF], g[CF::PF];

    RACE_DEV void load(const ScanParams &P, const Ctx &c, int t0, int hq, bool kv, int tid)
    {
        const int nv = min(CF::C, c.t_end - t0);
        if (kv) {
            tile_load<CF>(k, row_ptr(P.k, c.b, c.hk, t0), P.k.st, nv, tid);
            tile_load<CF>(v, row_ptr(P.v, c.b, c.hk, t0), P.v.st, nv, tid);
        }
        tile_load<CF>(q, row_ptr(P.q, c.b, hq, t0), P.q.st, nv, tid);
        tile_load<CF>(g, row_ptr(P.go, c.b, hq, t0), P.go.st, nv, tid);
    }

    // after storing step (t0, g): issue the loads of the following step, if any
    RACE_DEV void advance(const ScanParams &P, const Ctx &c, int t0, int g, int tid)
    {
        int g2 = g + 1, t2 = t0;
        if (g2 == P.G) {
            g2 = 0;
            t2 = t0 + CF::C;
        }
        if (t2 < c.t_end)
            load(P, c, t2, c.hk * P.G + g2, g2 == 0, tid);
    }
};

// ============================================================================ backward totals
// Forward-order pass over a block: dq (soft-hash backward of gpQ = gW/(A+eps)) and the
// block totals of W^T go (into ws2B) and of gA (into ws2A).
template <int ST, int DP, int KB, int NW, bool OUT_F32, bool G1>
__global__ __launch_bounds__(NW * 64) void race_fused_bwd_totals(const ScanParams P)
{
    using CF = FCfg<ST, DP, KB, NW>;
    constexpr int C = CF::C, NTH = CF::NTH, R = CF::R, MTC = CF::MTC;
    constexpr int LDX = CF::LDX, LDC = CF::LDC, LDS = CF::LDS, LDG = CF::LDG;
    using OT = typename std::conditional<OUT_F32, float, __bf16>::type;
    constexpr int LDO = DP + (OUT_F32 ? 4 : 8);
    __shared__ __align__(16) __bf16 sK[C][CF::LDQ];
    __shared__ __align__(16) __bf16 sQ[C][CF::LDQ];
    __shared__ __align__(16) __bf16 sV[C][LDX];
    __shared__ __align__(16) __bf16 sGO[C][LDX];
    __shared__ __align__(16) __bf16 sPK[C][LDS];   // rows [t][s]
    __shared__ __align__(16) __bf16 sPQ[C][LDS];
    __shared__ __align__(16) __bf16 sW[C][LDS];
    __shared__ __align__(16) __bf16 sMg[C][LDC];   // Mg as [t][tau]
    __shared__ __align__(16) __bf16 sStS[CF::NTS == NW ? 1 : ST][LDX];  // St rows when not in registers
    __shared__ __align__(16) float sGP[C][ST + 4];
    __shared__ __align__(16) __bf16 sGU[C][LDG];
    __shared__ __align__(16) OT sO[C][LDO];
    __shared__ __align__(16) float sA0[2][ST];
    __shared__ float sGAred[ST];

    const Ctx c = make_ctx(P, ST);
    const float coef = -2.0f * SH_LOG2E * P.inv_scale;  // soft-hash exponent factor
    const int tid = c.tid, lane = c.lane, wave = c.wave;
    __builtin_assume(wave >= 0 && wave < NW);  // (threadIdx.x < NW * 64): per-wave tile counts that divide evenly need no guard
    constexpr int TPW_P = (2 * CF::NPT + NW - 1) / NW;   // k then q projection tiles
    constexpr int TPW_S = (CF::NTS * CF::NTD + NW - 1) / NW;
    constexpr int TPW_A = (CF::NTS * MTC + NW - 1) / NW;
    // A-tiles [ST x C] (A^T, W, gW, gA per bucket tile ts and token tile tt). When the waves
    // and the bucket tiles match one to one (REG_ST), wave w owns bucket tile w for every token
    // tile and every head-dim tile of the state, so gW = go St^T takes St from registers.
    constexpr bool REG_ST = CF::NTS == NW;
    auto a_ts = [&](int i) { return REG_ST ? wave : (wave + i * NW) / MTC; };
    auto a_tt = [&](int i) { return REG_ST ? i : (wave + i * NW) % MTC; };
    auto a_ok = [&](int i) { return REG_ST || (wave + i * NW) < CF::NTS * MTC; };
    constexpr int TPW_O = (CF::NTD * MTC + NW - 1) / NW;
    constexpr int TPW_M = (MTC * MTC + NW - 1) / NW;
    FusedFrags<CF, DP, TPW_P> fr;
    fr.load(P, c.l0, c.Lt, lane, wave);
    BackFrags<CF, DP, TPW_O> bk;
    bk.load(P, c.l0, c.Lt, lane, wave, MTC);
    zero_lds_bf16(&sPK[0][0], C * LDS, tid, NTH);
    zero_lds_bf16(&sPQ[0][0], C * LDS, tid, NTH);
    zero_lds_bf16(&sGU[0][0], C * LDG, tid, NTH);
    for (int i = tid; i < ST; i += NTH)
        sGAred[i] = 0.0f;

    // St^T (lane: col s, rows d) at the block start, and dS^T totals
    const int64_t slot = (int64_t)c.z * (P.NB + 1) + c.blk;
    f32x4 accS[TPW_S], accD[TPW_S];
    {
        const float *wB = P.wsB + (slot * P.S_pad + c.s0) * P.DPw;
#pragma unroll
        for (int i = 0; i < TPW_S; ++i) {
            const int t = wave + i * NW;
            accS[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            accD[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (t < CF::NTS * CF::NTD) {
                const int d = (t / CF::NTS) * 16 + ((lane >> 4) << 2), s = (t % CF::NTS) * 16 + (lane & 15);
                accS[i] = *reinterpret_cast<const f32x4 *>(wB + (int64_t)s * P.DPw + d);
                if constexpr (!REG_ST)
                    st_vec4(&sStS[s][d], accS[i]);
            }
        }
        const float *wA = P.wsA + slot * P.S_pad + c.s0;
        for (int s = tid; s < ST; s += NTH)
            sA0[0][s] = wA[s] + P.eps;  // the carry holds A + eps
    }
    f32x4 accGA[TPW_A];
#pragma unroll
    for (int i = 0; i < TPW_A; ++i)
        accGA[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int G = G1 ? 1 : P.G;  // G1: one query head per kv head, the head loop folds away
    const int nsub = (c.t_end - c.t_begin + C - 1) / C;
    int prev_t0 = -1, prev_nv = 0, prev_h = 0;
    AccRows<C, DP, NTH> arQ;
    RowPrefetch<CF> pf;
    pf.load(P, c, c.t_begin, c.hk * G, true, tid);
    wait_vmem_all();
    f32x4 accI[TPW_A];  // 1/(A+eps), A^T tiles
    float thq[TPW_P][4], pq_[TPW_P][R];

    // Software pipeline over (sub-chunk, head) steps: the tail of a step (T4 soft-hash
    // backward of q, T5 dq, the dq rows out) runs in the barrier phases P0, P1, P2 of the next
    // step, so a step costs four barrier phases.
    // ---- T4: soft-hash backward of q -> gproj -> sGU ; (after the last head) St -> sStS
    auto tail4 = [&](bool st_rows) {
#pragma unroll
        for (int i = 0; i < TPW_P; ++i) {
            const int t = wave + i * NW;
            if (t >= CF::NPT && t < 2 * CF::NPT) {
                const int tq_ = t - CF::NPT;
                const int jt = tq_ / MTC, tt = tq_ % MTC;
                const int tok = tt * 16 + (lane & 15), table = jt * 4 + (lane >> 4);
                if (table < CF::LT) {
                    float gp[R], gproj[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int h = 0; h < R / 4; ++h) {
                        const f32x4 x = *reinterpret_cast<const f32x4 *>(&sGP[tok][table * R + 4 * h]);
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            gp[4 * h + e] = x[e];
                    }
                    softhash_bwd_ct<KB>(thq[i], pq_[i], gp, P.inv_scale, gproj);
                    bf16x4 w;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        w[e] = (__bf16)(e < KB ? gproj[e] : 0.0f);
                    *reinterpret_cast<bf16x4 *>(&sGU[tok][table * 4]) = w;
                }
            }
        }
        if (st_rows) {
#pragma unroll
            for (int i = 0; i < TPW_S; ++i) {
                const int t = wave + i * NW;
                if (t < CF::NTS * CF::NTD) {
                    const int d = (t / CF::NTS) * 16 + ((lane >> 4) << 2), s = (t % CF::NTS) * 16 + (lane & 15);
                    if constexpr (!REG_ST)
                        st_vec4(&sStS[s][d], accS[i]);
                }
            }
        }
    };
    // ---- T5: dq^T = P gproj^T -> sO
    auto tail5 = [&]() {
#pragma unroll
        for (int i = 0; i < TPW_O; ++i) {
            const int t = wave + i * NW;
            if (t < CF::NTD * MTC) {
                const int td = t / MTC, tt = t % MTC;
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                const __bf16 *pb = &sGU[0][0] + (tt * 16 + (lane & 15)) * LDG + (lane >> 4) * 8;
#pragma unroll
                for (int kb = 0; kb < (CF::LKP + 31) / 32; ++kb)
                    EngBF16::mma(acc, bk.f[i][kb], *reinterpret_cast<const bf16x8 *>(pb + kb * 32));
                const int d = td * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
                if constexpr (OUT_F32)
                    *reinterpret_cast<f32x4 *>(&sO[tok][d]) = acc;
                else
                    st_vec4(&sO[tok][d], acc);
            }
        }
    };

    for (int sc = 0; sc < nsub; ++sc) {
        const int t0 = c.t_begin + sc * C;
        const int nv = min(C, c.t_end - t0);
        const int cur = sc & 1, nxt = cur ^ 1;
        for (int g = 0; g < G; ++g) {
            const int hq = c.hk * G + g;
            const bool tail = prev_t0 >= 0;
            // ---- P0: rows of this (sub-chunk, head) into LDS (their loads were issued a step ago)
            //          | T4 of the previous step
            wait_vmem_all();
            if (g == 0) {
                tile_store_kq<CF>(&sK[0][0], pf.k, tid);
                tile_store_rows<CF>(&sV[0][0], pf.v, nv, tid);
            }
            tile_store_kq<CF>(&sQ[0][0], pf.q, tid);
            tile_store_rows<CF>(&sGO[0][0], pf.g, nv, tid);
            // (tiles one launch after another) the earlier tiles' sum of the previous step's dq
            // rows, stored in P2; issued before the row prefetch so that waiting for it does not
            // wait for the prefetch
            if constexpr (OUT_F32) {
                if (tail && P.dq.stage_f32)
                    arQ.load(P.dq, c.b, prev_h, prev_t0, prev_nv, tid);
            }
            pf.advance(P, c, t0, g, tid);
            if (tail)
                tail4(g == 0);
            __syncthreads();
            // ---- P1: soft-hash of k (first head) -> pK^T ; of q -> pQ (kept in registers)
            //          | T5 of the previous step
            if (tail)
                tail5();
#pragma unroll
            for (int i = 0; i < TPW_P; ++i) {
                const int t = wave + i * NW;
                const bool isk = t < CF::NPT;
                if (t < 2 * CF::NPT && (!isk || g == 0)) {
                    const int tq_ = isk ? t : t - CF::NPT;
                    const int jt = tq_ / MTC, tt = tq_ % MTC;
                    const f32x4 acc = proj_T<CF, DP, TPW_P>(fr, i, isk ? &sK[0][0] : &sQ[0][0], tt, lane);
                    const int tok = tt * 16 + (lane & 15), table = jt * 4 + (lane >> 4);
                    const bool ok = tok < nv && table < c.Lt;
                    float th[4], p[R];
                    softhash_fwd_ct<KB>(acc, coef, ok, th, p);
                    if (table < CF::LT) {
                        __bf16 *row = isk ? &sPK[tok][table * R] : &sPQ[tok][table * R];
#pragma unroll
                        for (int h = 0; h < R / 4; ++h) {
                            bf16x4 w;
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                w[e] = (__bf16)p[4 * h + e];
                            *reinterpret_cast<bf16x4 *>(row + 4 * h) = w;
                        }
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        thq[i][e] = th[e];
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        pq_[i][r] = p[r];
                }
            }
            __syncthreads();
            // ---- P2: A^T scan (first head) -> 1/(A+eps); W -> sW ; Mg -> sMg ; gW^T = St go^T
            //          | the previous step's dq rows out
            if (tail)
                store_out<OT, C, DP, LDO, NTH>(P.dq, c.b, prev_h, c.st, prev_t0, prev_nv, sO, arQ, tid);
            f32x4 accW[TPW_A], accG[TPW_A];
            // (REG_ST) pK^T of the wave's bucket tile: the operand of the A scan, gW and St, read once
            const bf16x8 fPK = ld_tr(&sPK[0][0], LDS, 0, (REG_ST ? wave : 0) * 16, lane);
#pragma unroll
            for (int i = 0; i < TPW_A; ++i) {
                accW[i] = f32x4{0.f, 0.f, 0.f, 0.f};
                accG[i] = f32x4{0.f, 0.f, 0.f, 0.f};
                if (a_ok(i)) {
                    const int ts = a_ts(i), tt = a_tt(i);
                    const int s = ts * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
                    if (g == 0) {
                        f32x4 a = *reinterpret_cast<const f32x4 *>(&sA0[cur][s]);
                        EngBF16::mma(a, REG_ST ? fPK : ld_tr(&sPK[0][0], LDS, 0, ts * 16, lane), fr.tri_of(tt));
                        if (tt == MTC - 1 && (lane & 15) == 15)
                            *reinterpret_cast<f32x4 *>(&sA0[nxt][s]) = a;
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            accI[i][e] = frcp(a[e]);
                    }
                    const bf16x4 q4 = *reinterpret_cast<const bf16x4 *>(&sPQ[tok][s]);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        accW[i][e] = (float)q4[e] * accI[i][e];
                    st_vec4(&sW[tok][s], accW[i]);
                    if constexpr (REG_ST) {
#pragma unroll
                        for (int kd = 0; kd < DP / 32; ++kd)
                            EngBF16::mma(accG[i], acc_pair(accS[2 * kd], accS[2 * kd + 1]),
                                         ld_pair(&sGO[0][0], LDX, tt * 16, 32 * kd, lane));
                    } else {
                        mma_ab<DP, LDX, LDX>(accG[i], &sStS[0][0], ts * 16, &sGO[0][0], tt * 16, lane);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < TPW_M; ++i) {
                const int t = wave + i * NW;
                if (t < MTC * MTC) {
                    const int tu = t / MTC, tt = t % MTC;  // rows tau, cols t
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    mma_ab<DP, LDX, LDX>(acc, &sV[0][0], tu * 16, &sGO[0][0], tt * 16, lane);
                    const int tau = tu * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (tau + e > tok)
                            acc[e] = 0.0f;
                    st_vec4(&sMg[tok][tau], acc);
                }
            }
            __syncthreads();
            // ---- P3: gW^T += pK^T Mg^T ; gpQ^T -> sGP ; gA ; dS^T += go^T W ; St^T += V^T pK (last head)
#pragma unroll
            for (int i = 0; i < TPW_A; ++i) {
                if (a_ok(i)) {
                    const int ts = a_ts(i), tt = a_tt(i);
                    const int s = ts * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
                    EngBF16::mma(accG[i], REG_ST ? fPK : ld_tr(&sPK[0][0], LDS, 0, ts * 16, lane),
                                 ld_k(&sMg[0][0], LDC, tt * 16, 0, lane));
                    f32x4 gpq;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        gpq[e] = accG[i][e] * accI[i][e];
                        accGA[i][e] -= gpq[e] * accW[i][e];
                    }
                    *reinterpret_cast<f32x4 *>(&sGP[tok][s]) = gpq;
                }
            }
            // (REG_ST) W^T of the wave's bucket tile, read once for its dS tiles
            const bf16x8 fW = ld_tr(&sW[0][0], LDS, 0, (REG_ST ? wave : 0) * 16, lane);
#pragma unroll
            for (int i = 0; i < TPW_S; ++i) {
                const int t = wave + i * NW;
                if (t < CF::NTS * CF::NTD) {
                    const int td = t / CF::NTS, ts = t % CF::NTS;
                    EngBF16::mma(accD[i], ld_tr(&sGO[0][0], LDX, 0, td * 16, lane),
                                 REG_ST ? fW : ld_tr(&sW[0][0], LDS, 0, ts * 16, lane));
                    if (g == G - 1)
                        EngBF16::mma(accS[i], ld_tr(&sV[0][0], LDX, 0, td * 16, lane),
                                     REG_ST ? fPK : ld_tr(&sPK[0][0], LDS, 0, ts * 16, lane));
                }
            }
            prev_t0 = t0;
            prev_nv = nv;
            prev_h = hq;
            __syncthreads();
        }
    }
    // tail of the last step
    tail4(false);
    __syncthreads();
    tail5();
    if constexpr (OUT_F32) {
        if (P.dq.stage_f32)
            arQ.load(P.dq, c.b, prev_h, prev_t0, prev_nv, tid);
    }
    __syncthreads();
    store_out<OT, C, DP, LDO, NTH>(P.dq, c.b, prev_h, c.st, prev_t0, prev_nv, sO, arQ, tid);

    // block totals: dS^T -> ws2B [s][d] ; gA (sum over tokens) -> ws2A
    float *wB = P.ws2B + (slot * P.S_pad + c.s0) * P.DPw;
#pragma unroll
    for (int i = 0; i < TPW_S; ++i) {
        const int t = wave + i * NW;
        if (t < CF::NTS * CF::NTD) {
            const int d = (t / CF::NTS) * 16 + ((lane >> 4) << 2), s = (t % CF::NTS) * 16 + (lane & 15);
            *reinterpret_cast<f32x4 *>(wB + (int64_t)s * P.DPw + d) = accD[i];
        }
    }
#pragma unroll
    for (int i = 0; i < TPW_A; ++i) {
        if (a_ok(i)) {
            const int ts = a_ts(i);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float v = accGA[i][e];
                v += __shfl_xor(v, 1);
                v += __shfl_xor(v, 2);
                v += __shfl_xor(v, 4);
                v += __shfl_xor(v, 8);
                if ((lane & 15) == 0)
                    atomicAdd(&sGAred[ts * 16 + ((lane >> 4) << 2) + e], v);
            }
        }
    }
    __syncthreads();
    float *wA = P.ws2A + slot * P.S_pad + c.s0;
    for (int s = tid; s < ST; s += NTH)
        wA[s] = sGAred[s];
}


// ============================================================================ backward main
// Forward-order pass over a block with the suffix states (dS, gAhat) shrinking by each
// sub-chunk's contribution (exact forward A and St, see race_scan_kernels.h):
//   gpK^T = gAhat + dS V^T + W^T Mg ,   gv^T = dS^T pK^T + go^T Mp^T
// then dk through the soft-hash backward of k and dv directly. Each matrix is held once in
// LDS, in the orientation its producer writes with vector stores; operands that need the
// other orientation are read with ld_tr.
//
// Software pipeline over sub-chunks: each sub-chunk is a head (H0 rows, H1 soft-hash, H2
// A/W/gW/Mg, H3, H4) and a tail (T5 gpK, T6 soft-hash backward of k and dv, T7 dk). The
// tail of sub-chunk i runs in the barrier phases of H0, H1, H2 of sub-chunk i+1, so a
// sub-chunk costs five barrier phases. Arrays that both sides touch are double buffered by
// sub-chunk parity (v rows, pK) or kept apart (dS^T, the dk and dv staging).
template <int ST, int DP, int KB, int NW, bool OUT_F32, bool G1>
__global__ __launch_bounds__(NW * 64) void race_fused_bwd_main(const ScanParams P)
{
    using CF = FCfg<ST, DP, KB, NW>;
    constexpr int C = CF::C, NTH = CF::NTH, R = CF::R, MTC = CF::MTC;
    constexpr int LDX = CF::LDX, LDC = CF::LDC, LDS = CF::LDS, LDG = CF::LDG, LDF = ST + 4;
    using OT = typename std::conditional<OUT_F32, float, __bf16>::type;
    constexpr int LDO = DP + (OUT_F32 ? 4 : 8);
    // uF holds gpK rows in fp32 (T5 -> T6) and the gA^T hi/lo parts (H3 -> H4): disjoint phases
    constexpr int SZ_PQ = C * LDS * 2;
    constexpr int SZ_F = C * LDF * 4 > 2 * SZ_PQ ? C * LDF * 4 : 2 * SZ_PQ;
    __shared__ __align__(16) char uF[SZ_F];
    float(*sF)[LDF] = reinterpret_cast<float(*)[LDF]>(uF);
    __bf16(*sGAh)[LDS] = reinterpret_cast<__bf16(*)[LDS]>(uF);
    __bf16(*sGAl)[LDS] = reinterpret_cast<__bf16(*)[LDS]>(uF + SZ_PQ);
    __shared__ __align__(16) __bf16 sK[C][CF::LDQ];
    __shared__ __align__(16) __bf16 sQ[C][CF::LDQ];
    __shared__ __align__(16) __bf16 sV[2][C][LDX];   // by sub-chunk parity
    // go rows; two buffers by step parity where the go^T Mp^T product of a step is deferred to
    // the next step's first phase (one wave per bucket tile)
    __shared__ __align__(16) __bf16 sGO[CF::NTS == NW ? 2 : 1][C][LDX];
    __shared__ __align__(16) __bf16 sPK[2][C][LDS];  // by sub-chunk parity
    __shared__ __align__(16) __bf16 sPQ[C][LDS];
    __shared__ __align__(16) __bf16 sW[C][LDS];
    __shared__ __align__(16) __bf16 sdSt[DP][LDS];   // dS^T [d][s]
    __shared__ __align__(16) __bf16 sMg[C][LDC];     // Mg as [tau][t]
    __shared__ __align__(16) __bf16 sMp[C][LDC];     // Mp as [tau][t]
    __shared__ __align__(16) __bf16 sStS[CF::NTS == NW ? 1 : ST][LDX];  // St rows when not in registers
    __shared__ __align__(16) __bf16 sGU[C][LDG];
    __shared__ __align__(16) OT sOk[C][LDO];
    __shared__ __align__(16) OT sOv[C][LDO];
    __shared__ __align__(16) float sA0[2][ST];
    __shared__ __align__(16) float sGAe[2][ST];

    const Ctx c = make_ctx(P, ST);
    const float coef = -2.0f * SH_LOG2E * P.inv_scale;  // soft-hash exponent factor
    const int tid = c.tid, lane = c.lane, wave = c.wave;
    __builtin_assume(wave >= 0 && wave < NW);  // (threadIdx.x < NW * 64): per-wave tile counts that divide evenly need no guard
    constexpr int TPW_P = (2 * CF::NPT + NW - 1) / NW;
    constexpr int TPW_S = (CF::NTS * CF::NTD + NW - 1) / NW;
    constexpr int TPW_A = (CF::NTS * MTC + NW - 1) / NW;
    // A-tiles [ST x C] (A^T, W, gW, gA per bucket tile ts and token tile tt). When the waves
    // and the bucket tiles match one to one (REG_ST), wave w owns bucket tile w for every token
    // tile and every head-dim tile of the state, so gW = go St^T takes St from registers.
    constexpr bool REG_ST = CF::NTS == NW;
    // REG_ST: dS^T goes to LDS at the end of H3 and gv += go^T Mp^T runs in the next step's H0,
    // so a step has four barrier phases; otherwise H4 holds both and the MFMA gA suffix scan
    constexpr bool DEFER_GV = REG_ST;
    auto a_ts = [&](int i) { return REG_ST ? wave : (wave + i * NW) / MTC; };
    auto a_tt = [&](int i) { return REG_ST ? i : (wave + i * NW) % MTC; };
    auto a_ok = [&](int i) { return REG_ST || (wave + i * NW) < CF::NTS * MTC; };
    constexpr int TPW_O = (CF::NTD * MTC + NW - 1) / NW;
    constexpr int TPW_M = (MTC * MTC + NW - 1) / NW;
    // dv tiles live on the last GVW waves, so that the soft-hash backward of k (on the
    // first NPT waves) and the final dv product run side by side
    constexpr int GVW = NW - (CF::NPT < NW / 2 ? CF::NPT : NW / 2);
    constexpr int TPW_V = (CF::NTD * MTC + GVW - 1) / GVW;
    const int wv = wave - (NW - GVW);
    FusedFrags<CF, DP, TPW_P> fr;
    fr.load(P, c.l0, c.Lt, lane, wave);
    BackFrags<CF, DP, TPW_O> bk;
    bk.load(P, c.l0, c.Lt, lane, wave, MTC);
    zero_lds_bf16(&sPK[0][0][0], 2 * C * LDS, tid, NTH);
    zero_lds_bf16(&sGU[0][0], C * LDG, tid, NTH);

    // St^T at the block start (lane: col s, rows d); suffix dS from the block start
    // (accD, lane: col d, rows s).
    const int64_t slot = (int64_t)c.z * (P.NB + 1) + c.blk;
    f32x4 accS[TPW_S], accD[TPW_S];
    {
        const float *wB = P.wsB + (slot * P.S_pad + c.s0) * P.DPw;
        const float *wB2 = P.ws2B + (slot * P.S_pad + c.s0) * P.DPw;
#pragma unroll
        for (int i = 0; i < TPW_S; ++i) {
            const int t = wave + i * NW;
            accS[i] = accD[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (t < CF::NTS * CF::NTD) {
                const int td = t / CF::NTS, ts = t % CF::NTS;
                const int d = td * 16 + ((lane >> 4) << 2), s = ts * 16 + (lane & 15);
                accS[i] = *reinterpret_cast<const f32x4 *>(wB + (int64_t)s * P.DPw + d);
                if constexpr (!REG_ST)
                    st_vec4(&sStS[s][d], accS[i]);
                const int s2 = ts * 16 + ((lane >> 4) << 2), d2 = td * 16 + (lane & 15);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    accD[i][e] = wB2[(int64_t)(s2 + e) * P.DPw + d2];
            }
        }
        const float *wA = P.wsA + slot * P.S_pad + c.s0;
        const float *wA2 = P.ws2A + slot * P.S_pad + c.s0;
        for (int s = tid; s < ST; s += NTH) {
            sA0[0][s] = wA[s] + P.eps;  // the carry holds A + eps
            sGAe[0][s] = wA2[s];
        }
    }

    const int G = G1 ? 1 : P.G;  // G1: one query head per kv head, the head loop folds away
    const int nsub = (c.t_end - c.t_begin + C - 1) / C;
    RowPrefetch<CF> pf;
    pf.load(P, c, c.t_begin, c.hk * G, true, tid);
    wait_vmem_all();
    f32x4 accI[TPW_A], accPK[TPW_A], accV[TPW_V], accGA[TPW_A];
    float thk[TPW_P][4];
#pragma unroll
    for (int i = 0; i < TPW_A; ++i)
        accPK[i] = accGA[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < TPW_V; ++i)
        accV[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    // ---- gv^T += go^T Mp^T of a step (go rows in buffer gbuf)
    auto gv_mp = [&](int gbuf) {
#pragma unroll
        for (int i = 0; i < TPW_V; ++i) {
            const int t = wv + i * GVW;
            if (wv >= 0 && t < CF::NTD * MTC)
                EngBF16::mma(accV[i], ld_tr(&sGO[gbuf][0][0], LDX, 0, (t / MTC) * 16, lane),
                             ld_k(&sMp[0][0], LDC, (t % MTC) * 16, 0, lane));
        }
    };
    // ---- T5 (sub-chunk buffer pb): gpK^T += dS V^T + gAhat -> sF ; St -> sStS
    auto tail5 = [&](int pb) {
#pragma unroll
        for (int i = 0; i < TPW_A; ++i) {
            if (a_ok(i)) {
                const int ts = a_ts(i), tt = a_tt(i);
                const int s = ts * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
#pragma unroll
                for (int kd = 0; kd < DP; kd += 32)
                    EngBF16::mma(accPK[i], ld_tr(&sdSt[0][0], LDS, kd, ts * 16, lane),
                                 ld_k(&sV[pb][0][0], LDX, tt * 16, kd, lane));
                f32x4 x;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    x[e] = accPK[i][e] + accGA[i][e];
                *reinterpret_cast<f32x4 *>(&sF[tok][s]) = x;
                accPK[i] = accGA[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
#pragma unroll
        for (int i = 0; i < TPW_S; ++i) {
            const int t = wave + i * NW;
            if (t < CF::NTS * CF::NTD) {
                const int d = (t / CF::NTS) * 16 + ((lane >> 4) << 2), s = (t % CF::NTS) * 16 + (lane & 15);
                if constexpr (!REG_ST)
                    st_vec4(&sStS[s][d], accS[i]);
            }
        }
    };
    // ---- T6 (buffer pb, nv_ valid tokens, tanh of the k projections thkp): gv^T += dS^T pK^T -> sOv ;
    //      soft-hash backward of k -> sGU
    auto tail6 = [&](int pb, int nv_, const float (&thkp)[TPW_P][4]) {
#pragma unroll
        for (int i = 0; i < TPW_V; ++i) {
            const int t = wv + i * GVW;
            if (wv >= 0 && t < CF::NTD * MTC) {
                const int td = t / MTC, tt = t % MTC;
                mma_ab<ST, LDS, LDS>(accV[i], &sdSt[0][0], td * 16, &sPK[pb][0][0], tt * 16, lane);
                const int d = td * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
                if constexpr (OUT_F32)
                    *reinterpret_cast<f32x4 *>(&sOv[tok][d]) = accV[i];
                else
                    st_vec4(&sOv[tok][d], accV[i]);
            }
            accV[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int i = 0; i < TPW_P; ++i) {
            const int t = wave + i * NW;
            if (t < CF::NPT) {
                const int jt = t / MTC, tt = t % MTC;
                const int tok = tt * 16 + (lane & 15), table = jt * 4 + (lane >> 4);
                if (table < CF::LT) {
                    float gp[R], gproj[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int h = 0; h < R / 4; ++h) {
                        const f32x4 x = *reinterpret_cast<const f32x4 *>(&sF[tok][table * R + 4 * h]);
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            gp[4 * h + e] = x[e];
                    }
                    float pk[R];
                    probs_from_th<KB>(thkp[i], coef, tok < nv_ && table < c.Lt ? 1.0f : 0.0f, pk);
                    softhash_bwd_ct<KB>(thkp[i], pk, gp, P.inv_scale, gproj);
                    bf16x4 w;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        w[e] = (__bf16)(e < KB ? gproj[e] : 0.0f);
                    *reinterpret_cast<bf16x4 *>(&sGU[tok][table * 4]) = w;
                }
            }
        }
    };
    // ---- T7: dk^T = P gproj^T -> sOk
    auto tail7 = [&]() {
#pragma unroll
        for (int i = 0; i < TPW_O; ++i) {
            const int t = wave + i * NW;
            if (t < CF::NTD * MTC) {
                const int td = t / MTC, tt = t % MTC;
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                const __bf16 *pb = &sGU[0][0] + (tt * 16 + (lane & 15)) * LDG + (lane >> 4) * 8;
#pragma unroll
                for (int kb = 0; kb < (CF::LKP + 31) / 32; ++kb)
                    EngBF16::mma(acc, bk.f[i][kb], *reinterpret_cast<const bf16x8 *>(pb + kb * 32));
                const int d = td * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
                if constexpr (OUT_F32)
                    *reinterpret_cast<f32x4 *>(&sOk[tok][d]) = acc;
                else
                    st_vec4(&sOk[tok][d], acc);
            }
        }
    };

    int prev_t0 = -1, prev_nv = 0, gb = 0;
    AccRows<C, DP, NTH> arK, arV;
    for (int sc = 0; sc < nsub; ++sc) {
        const int t0 = c.t_begin + sc * C;
        const int nv = min(C, c.t_end - t0);
        const int cur = sc & 1, nxt = cur ^ 1;
        const bool tail = sc > 0;  // the previous sub-chunk's tail runs in H0..H2 (first head)
        for (int g = 0; g < G; ++g) {
            // ---- H0: rows into LDS (their loads were issued a step ago) | T5 of the previous sub-chunk
            wait_vmem_all();
            if (g == 0) {
                tile_store_kq<CF>(&sK[0][0], pf.k, tid);
                tile_store_rows<CF>(&sV[cur][0][0], pf.v, nv, tid);
            }
            tile_store_kq<CF>(&sQ[0][0], pf.q, tid);
            tile_store_rows<CF>(&sGO[gb][0][0], pf.g, nv, tid);
            // (tiles one launch after another) the earlier tiles' sums of the previous sub-chunk's
            // dk and dv rows, stored in H3; issued before the row prefetch
            if constexpr (OUT_F32) {
                if (g == 0 && tail && P.dk.stage_f32) {
                    arK.load(P.dk, c.b, c.hk, prev_t0, prev_nv, tid);
                    arV.load(P.dv, c.b, c.hk, prev_t0, prev_nv, tid);
                }
            }
            pf.advance(P, c, t0, g, tid);
            if constexpr (DEFER_GV) {
                if (sc > 0 || g > 0)
                    gv_mp(gb ^ 1);  // the previous step's go^T Mp^T
            }
            if (g == 0 && tail)
                tail5(nxt);
            __syncthreads();
            // ---- H1: soft-hash of k (first head) -> pK ; of q -> pQ   (rows [t][s])
            //          | T6 of the previous sub-chunk
            if (g == 0 && tail) {
                float thkp[TPW_P][4];
#pragma unroll
                for (int i = 0; i < TPW_P; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        thkp[i][e] = thk[i][e];
                tail6(nxt, prev_nv, thkp);
            }
#pragma unroll
            for (int i = 0; i < TPW_P; ++i) {
                const int t = wave + i * NW;
                const bool isk = t < CF::NPT;
                if (t < 2 * CF::NPT && (!isk || g == 0)) {
                    const int tq_ = isk ? t : t - CF::NPT;
                    const int jt = tq_ / MTC, tt = tq_ % MTC;
                    const f32x4 acc = proj_T<CF, DP, TPW_P>(fr, i, isk ? &sK[0][0] : &sQ[0][0], tt, lane);
                    const int tok = tt * 16 + (lane & 15), table = jt * 4 + (lane >> 4);
                    const bool ok = tok < nv && table < c.Lt;
                    float th[4], p[R];
                    softhash_fwd_ct<KB>(acc, coef, ok, th, p);
                    if (table < CF::LT) {
                        __bf16 *row = isk ? &sPK[cur][tok][table * R] : &sPQ[tok][table * R];
#pragma unroll
                        for (int h = 0; h < R / 4; ++h) {
                            bf16x4 w;
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                w[e] = (__bf16)p[4 * h + e];
                            *reinterpret_cast<bf16x4 *>(row + 4 * h) = w;
                        }
                    }
                    if (isk) {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            thk[i][e] = th[e];
                    }
                }
            }
            __syncthreads();
            // ---- H2: A^T (first head) ; W -> sW ; gW^T = St go^T ; Mg -> sMg | T7 of the previous sub-chunk
            if (g == 0 && tail)
                tail7();
            f32x4 accW[TPW_A], accG[TPW_A];
            // (REG_ST) pK^T of the wave's bucket tile: the operand of the A scan, gW and St, read once
            const bf16x8 fPK = ld_tr(&sPK[cur][0][0], LDS, 0, (REG_ST ? wave : 0) * 16, lane);
#pragma unroll
            for (int i = 0; i < TPW_A; ++i) {
                accW[i] = accG[i] = f32x4{0.f, 0.f, 0.f, 0.f};
                if (a_ok(i)) {
                    const int ts = a_ts(i), tt = a_tt(i);
                    const int s = ts * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
                    if (g == 0) {
                        f32x4 a = *reinterpret_cast<const f32x4 *>(&sA0[cur][s]);
                        EngBF16::mma(a, REG_ST ? fPK : ld_tr(&sPK[cur][0][0], LDS, 0, ts * 16, lane), fr.tri_of(tt));
                        if (tt == MTC - 1 && (lane & 15) == 15)
                            *reinterpret_cast<f32x4 *>(&sA0[nxt][s]) = a;
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            accI[i][e] = frcp(a[e]);
                    }
                    const bf16x4 q4 = *reinterpret_cast<const bf16x4 *>(&sPQ[tok][s]);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        accW[i][e] = (float)q4[e] * accI[i][e];
                    st_vec4(&sW[tok][s], accW[i]);
                    if constexpr (REG_ST) {
#pragma unroll
                        for (int kd = 0; kd < DP / 32; ++kd)
                            EngBF16::mma(accG[i], acc_pair(accS[2 * kd], accS[2 * kd + 1]),
                                         ld_pair(&sGO[gb][0][0], LDX, tt * 16, 32 * kd, lane));
                    } else {
                        mma_ab<DP, LDX, LDX>(accG[i], &sStS[0][0], ts * 16, &sGO[gb][0][0], tt * 16, lane);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < TPW_M; ++i) {
                const int t = wave + i * NW;
                if (t < MTC * MTC) {
                    // Mg[t][tau] = go_t . v_tau (tau <= t): rows t (tile ta), cols tau (tile tb)
                    const int ta = t / MTC, tb = t % MTC;
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    mma_ab<DP, LDX, LDX>(acc, &sGO[gb][0][0], ta * 16, &sV[cur][0][0], tb * 16, lane);
                    const int r0 = ta * 16 + ((lane >> 4) << 2), c0 = tb * 16 + (lane & 15);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (c0 > r0 + e)
                            acc[e] = 0.0f;
                    st_vec4(&sMg[c0][r0], acc);
                }
            }
            __syncthreads();
            // ---- H3: gW^T += pK^T Mg^T ; gA^T ; gpK^T += W^T Mg ; Mp -> sMp ;
            //          dS -= W^T go ; St^T += V^T pK (last head) ; gA^T hi/lo -> [tau][s] ;
            //          previous sub-chunk's dk, dv out
            if (g == 0 && tail) {
                store_out<OT, C, DP, LDO, NTH>(P.dk, c.b, c.hk, c.st, prev_t0, prev_nv, sOk, arK, tid);
                store_out<OT, C, DP, LDO, NTH>(P.dv, c.b, c.hk, c.st, prev_t0, prev_nv, sOv, arV, tid);
            }
            // (REG_ST) W^T of the wave's bucket tile: the operand of gpK and dS, read once
            const bf16x8 fW = ld_tr(&sW[0][0], LDS, 0, (REG_ST ? wave : 0) * 16, lane);
#pragma unroll
            for (int i = 0; i < TPW_A; ++i) {
                if (a_ok(i)) {
                    const int ts = a_ts(i), tt = a_tt(i);
                    EngBF16::mma(accG[i], REG_ST ? fPK : ld_tr(&sPK[cur][0][0], LDS, 0, ts * 16, lane),
                                 ld_tr(&sMg[0][0], LDC, 0, tt * 16, lane));
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        accGA[i][e] -= accG[i][e] * accI[i][e] * accW[i][e];
                    EngBF16::mma(accPK[i], REG_ST ? fW : ld_tr(&sW[0][0], LDS, 0, ts * 16, lane),
                                 ld_k(&sMg[0][0], LDC, tt * 16, 0, lane));
                }
            }
            if constexpr (REG_ST) {
                if (g == G - 1) {
                    // gAhat_t = gAhat_start - sum_{tau < t} gA_tau. Wave w holds bucket tile w for
                    // both token tiles, and a token tile's 16 tokens lie along the 16 lanes of a DPP
                    // row: fp32 row scans, with token tile 0's row total carried into tile 1; the
                    // sub-chunk total seeds the next sub-chunk.
                    const int s = wave * 16 + ((lane >> 4) << 2);
                    const f32x4 g0 = *reinterpret_cast<const f32x4 *>(&sGAe[cur][s]);
                    f32x4 carry = {0.f, 0.f, 0.f, 0.f}, gend;
#pragma unroll
                    for (int i = 0; i < TPW_A; ++i) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float sc = row_scan16(accGA[i][e]);
                            const float inc = i == 0 ? sc : sc + carry[e];  // (no "+ 0.0f" to issue)
                            gend[e] = g0[e] - inc;
                            accGA[i][e] += gend[e];
                            if (i + 1 < TPW_A)
                                carry[e] = row_bcast15(inc);
                        }
                    }
                    if ((lane & 15) == 15)
                        *reinterpret_cast<f32x4 *>(&sGAe[nxt][s]) = gend;
                }
            }
#pragma unroll
            for (int i = 0; i < TPW_M; ++i) {
                const int t = wave + i * NW;
                if (t < MTC * MTC) {
                    // Mp[tau][t] = pK_tau . W_t (t >= tau): rows t (tile ta), cols tau (tile tb)
                    const int ta = t / MTC, tb = t % MTC;
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                    mma_ab<ST, LDS, LDS>(acc, &sW[0][0], ta * 16, &sPK[cur][0][0], tb * 16, lane);
                    const int r0 = ta * 16 + ((lane >> 4) << 2), c0 = tb * 16 + (lane & 15);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (r0 + e < c0)
                            acc[e] = 0.0f;
                    st_vec4(&sMp[c0][r0], acc);
                }
            }
            const bf16x8 fWn = EngBF16::neg(fW);
#pragma unroll
            for (int i = 0; i < TPW_S; ++i) {
                const int t = wave + i * NW;
                if (t < CF::NTS * CF::NTD) {
                    const int td = t / CF::NTS, ts = t % CF::NTS;
                    // dS[s][d] -= sum_t W[t][s] go[t][d]   (accD: rows s of tile ts, cols d of td)
                    EngBF16::mma(accD[i], REG_ST ? fWn : EngBF16::neg(ld_tr(&sW[0][0], LDS, 0, ts * 16, lane)),
                                 ld_tr(&sGO[gb][0][0], LDX, 0, td * 16, lane));
                    // St^T[d][s] += sum_t V[t][d] pK[t][s]
                    if (g == G - 1)
                        EngBF16::mma(accS[i], ld_tr(&sV[cur][0][0], LDX, 0, td * 16, lane),
                                     REG_ST ? fPK : ld_tr(&sPK[cur][0][0], LDS, 0, ts * 16, lane));
                }
            }
            if constexpr (!REG_ST) {
#pragma unroll
                for (int i = 0; i < TPW_A; ++i) {
                    if (a_ok(i) && g == G - 1) {
                        // gA^T as a bf16 hi/lo pair, rows [tau][s], for the suffix-scan MFMA
                        const int ts = a_ts(i), tt = a_tt(i);
                        const int s = ts * 16 + ((lane >> 4) << 2), tok = tt * 16 + (lane & 15);
                        f32x4 lo;
                        bf16x4 hi;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            hi[e] = (__bf16)accGA[i][e];
                            lo[e] = accGA[i][e] - (float)hi[e];
                        }
                        *reinterpret_cast<bf16x4 *>(&sGAh[tok][s]) = hi;
                        st_vec4(&sGAl[tok][s], lo);
                    }
                }
            }
            if (DEFER_GV && g == G - 1) {
                // dS^T -> sdSt (last read in H1, two barriers ago; next read in T5)
#pragma unroll
                for (int i = 0; i < TPW_S; ++i) {
                    const int t = wave + i * NW;
                    if (t < CF::NTS * CF::NTD) {
                        const int td = t / CF::NTS, ts = t % CF::NTS;
                        const int s2 = ts * 16 + ((lane >> 4) << 2), d2 = td * 16 + (lane & 15);
                        st_vec4(&sdSt[d2][s2], accD[i]);
                    }
                }
            }
            __syncthreads();
            if constexpr (DEFER_GV) {
                gb ^= 1;
                continue;
            }
            // ---- H4: gv^T += go^T Mp^T ; (last head) dS^T -> sdSt, gAhat scan
            gv_mp(0);
            if (g == G - 1) {
#pragma unroll
                for (int i = 0; i < TPW_S; ++i) {
                    const int t = wave + i * NW;
                    if (t < CF::NTS * CF::NTD) {
                        const int td = t / CF::NTS, ts = t % CF::NTS;
                        const int s2 = ts * 16 + ((lane >> 4) << 2), d2 = td * 16 + (lane & 15);
                        st_vec4(&sdSt[d2][s2], accD[i]);
                    }
                }
                // (bucket tiles spread over waves) gAhat_t = gAhat_start - sum_{tau < t} gA_tau:
                // the inclusive sum runs on the MFMA (hi + lo parts, ~16-bit mantissa per term,
                // fp32 accumulation) and the own term is added back in fp32; the sub-chunk total
                // seeds the next sub-chunk.
#pragma unroll
                for (int i = 0; i < TPW_A; ++i) {
                    if (!REG_ST && a_ok(i)) {
                        const int ts = a_ts(i), tt = a_tt(i);
                        const int s = ts * 16 + ((lane >> 4) << 2);
                        f32x4 inc = {0.f, 0.f, 0.f, 0.f};
                        const bf16x8 tri = fr.tri_of(tt);
                        EngBF16::mma(inc, ld_tr(&sGAh[0][0], LDS, 0, ts * 16, lane), tri);
                        EngBF16::mma(inc, ld_tr(&sGAl[0][0], LDS, 0, ts * 16, lane), tri);
                        const f32x4 g0 = *reinterpret_cast<const f32x4 *>(&sGAe[cur][s]);
                        f32x4 gend;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            gend[e] = g0[e] - inc[e];
                            accGA[i][e] += gend[e];
                        }
                        if (tt == MTC - 1 && (lane & 15) == 15)
                            *reinterpret_cast<f32x4 *>(&sGAe[nxt][s]) = gend;
                    }
                }
            }
            __syncthreads();
        }
        prev_t0 = t0;
        prev_nv = nv;
    }
    // tail of the last sub-chunk
    const int pb = (nsub - 1) & 1;
    if constexpr (DEFER_GV)
        gv_mp(gb ^ 1);  // the last step's go^T Mp^T
    tail5(pb);
    __syncthreads();
    tail6(pb, prev_nv, thk);
    __syncthreads();
    tail7();
    if constexpr (OUT_F32) {
        if (P.dk.stage_f32) {
            arK.load(P.dk, c.b, c.hk, prev_t0, prev_nv, tid);
            arV.load(P.dv, c.b, c.hk, prev_t0, prev_nv, tid);
        }
    }
    __syncthreads();
    store_out<OT, C, DP, LDO, NTH>(P.dk, c.b, c.hk, c.st, prev_t0, prev_nv, sOk, arK, tid);
    store_out<OT, C, DP, LDO, NTH>(P.dv, c.b, c.hk, c.st, prev_t0, prev_nv, sOv, arV, tid);
}

}  // namespace race
