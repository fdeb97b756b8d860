// Small kernels around the chunked scan:
//   race_block_scan        prefix / suffix scan of block states (fp64 running sums)
//   race_reduce_partials   sum of per-bucket-tile partial outputs
//   race_softhash_fwd      probs [N,T,L*R] from x [B,H,T,D] (scaling/race_common.py:36-73)
//   race_softhash_bwd      dx from d(probs) (torch autograd of the same map)
//   race_decode_step       fused single-token GQA decode with carried state
//   race_state_extract     final (A, B) state of a forward pass -> decode state
#include "race_decode.h"
#include "race_device.h"
#include "race_launch.h"
#include "race_softhash.h"

namespace race {

// ============================================================================ block scan
// One workgroup owns SCAN_COLS consecutive state elements of one stream and walks the
// blocks in super-chunks of SEGS * SEG blocks. Each thread loads one segment of SEG blocks
// at once (independent loads, one memory latency per super-chunk), the segment totals are
// combined through LDS, and each thread writes its segment's running sums from its offset.
// Sums run in fp64 and are rounded once per output. (SEGS, SEG) follow the block count, so a
// scan over few blocks launches few threads.
//   rev = 0: slot b <- sum_{b' < b} x_b' (exclusive), slot NB <- total
//   rev = 1: slot b <- sum_{b' >= b} x_b' (inclusive suffix), slot NB <- 0
// With LO, every value is the pair (hi, lo) of a double-float (hi in ws, lo at the same offset in
// the lo array): the inputs are read as hi + lo and the sums are written back as such pairs, so a
// block total carried in fp64 by its producer reaches the consumer with ~48 mantissa bits.
constexpr int SCAN_COLS = 64;

// One launch scans two workspaces of the same block count: (wsB, elemsB) with the first
// ceil(elemsB / SCAN_COLS) workgroups along x, (wsA, elemsA) with the rest.
template <bool REV, bool LO, int SEGS, int SEG>
__global__ __launch_bounds__(SCAN_COLS *SEGS) void race_block_scan(float *wsB, int64_t elemsB, float *wsA,
                                                                  int64_t elemsA, float *loB, float *loA, int NB)
{
    __shared__ double tot[SEGS][SCAN_COLS];
    const int col = threadIdx.x % SCAN_COLS, seg = threadIdx.x / SCAN_COLS;
    const int nbB = (int)((elemsB + SCAN_COLS - 1) / SCAN_COLS);
    const bool isB = (int)blockIdx.x < nbB;
    float *ws = isB ? wsB : wsA;
    float *lo = isB ? loB : loA;
    const int64_t elems = isB ? elemsB : elemsA;
    const int64_t e = (int64_t)(isB ? blockIdx.x : blockIdx.x - nbB) * SCAN_COLS + col;
    const bool live = e < elems;
    // loads use a clamped column and block index (always inside this stream's workspace), so
    // they are unconditional and all SEG of them are in flight together; addresses are formed
    // per load, so no per-block pointer stays live
    const int64_t ec = live ? e : elems - 1;
    float *base = ws + (int64_t)blockIdx.y * (NB + 1) * elems;
    float *lbase = LO ? lo + (int64_t)blockIdx.y * (NB + 1) * elems : nullptr;
    constexpr int SUPER = SEGS * SEG;
    double carry = 0.0;
    for (int c0 = 0; c0 < NB; c0 += SUPER) {
        // block index of this thread's i-th element (ascending, or descending when REV)
        const int first = REV ? NB - 1 - c0 - seg * SEG : c0 + seg * SEG;
        double x[SEG];
#pragma unroll
        for (int i = 0; i < SEG; ++i) {
            const int b = REV ? first - i : first + i;
            const int bc = REV ? max(b, 0) : min(b, NB - 1);
            x[i] = (double)base[(int64_t)bc * elems + ec];
            if (LO)
                x[i] += (double)lbase[(int64_t)bc * elems + ec];
        }
#pragma unroll
        for (int i = 0; i < SEG; ++i) {
            const int b = REV ? first - i : first + i;
            if (REV ? b < 0 : b >= NB)
                x[i] = 0.0;
        }
        double t = 0.0;
#pragma unroll
        for (int i = 0; i < SEG; ++i)
            t += x[i];
        if (SEGS > 1) {
            tot[seg][col] = t;
            __syncthreads();
        }
        double run = carry, all = t;
        if (SEGS > 1) {
            all = 0.0;
#pragma unroll
            for (int j = 0; j < SEGS; ++j) {
                const double v = tot[j][col];
                if (j < seg)
                    run += v;
                all += v;
            }
        }
        carry += all;
#pragma unroll
        for (int i = 0; i < SEG; ++i) {
            const int b = REV ? first - i : first + i;
            const bool ok = live && (REV ? b >= 0 : b < NB);
            if (REV)
                run += x[i];
            if (ok) {
                const float hi = (float)run;
                base[(int64_t)b * elems + e] = hi;
                if (LO)
                    lbase[(int64_t)b * elems + e] = (float)(run - (double)hi);
            }
            if (!REV)
                run += x[i];
        }
        if (SEGS > 1)
            __syncthreads();
    }
    if (live && seg == 0) {
        const float hi = REV ? 0.0f : (float)carry;
        base[(int64_t)NB * elems + e] = hi;
        if (LO)
            lbase[(int64_t)NB * elems + e] = REV ? 0.0f : (float)(carry - (double)hi);
    }
}

template <bool REV, bool LO, int SEGS, int SEG>
static void launch_scan_cfg(dim3 grid, float *wsB, int64_t elemsB, float *wsA, int64_t elemsA, float *loB,
                            float *loA, int NB, hipStream_t s)
{
    hipLaunchKernelGGL((race_block_scan<REV, LO, SEGS, SEG>), grid, dim3(SCAN_COLS * SEGS), 0, s, wsB, elemsB, wsA,
                       elemsA, loB, loA, NB);
}

template <bool REV, bool LO>
static void launch_scan_dir(dim3 grid, float *wsB, int64_t elemsB, float *wsA, int64_t elemsA, float *loB,
                            float *loA, int NB, hipStream_t s)
{
    if (NB <= 8)
        launch_scan_cfg<REV, LO, 1, 8>(grid, wsB, elemsB, wsA, elemsA, loB, loA, NB, s);
    else if (NB <= 32)
        launch_scan_cfg<REV, LO, 4, 8>(grid, wsB, elemsB, wsA, elemsA, loB, loA, NB, s);
    else if (NB <= 128)
        launch_scan_cfg<REV, LO, 16, 8>(grid, wsB, elemsB, wsA, elemsA, loB, loA, NB, s);
    else  // super-chunks of 256 blocks (32 loads per thread would not fit the registers)
        launch_scan_cfg<REV, LO, 16, 16>(grid, wsB, elemsB, wsA, elemsA, loB, loA, NB, s);
}

hipError_t launch_block_scan(float *wsB, int64_t elemsB, float *wsA, int64_t elemsA, int NB, int Z, int rev,
                             hipStream_t s, float *loB, float *loA)
{
    const dim3 grid((unsigned)((elemsB + SCAN_COLS - 1) / SCAN_COLS + (elemsA + SCAN_COLS - 1) / SCAN_COLS),
                    (unsigned)Z);
    if ((loB == nullptr) != (loA == nullptr))
        return hipErrorInvalidValue;
    if (loB) {
        if (rev)
            launch_scan_dir<true, true>(grid, wsB, elemsB, wsA, elemsA, loB, loA, NB, s);
        else
            launch_scan_dir<false, true>(grid, wsB, elemsB, wsA, elemsA, loB, loA, NB, s);
    } else if (rev) {
        launch_scan_dir<true, false>(grid, wsB, elemsB, wsA, elemsA, nullptr, nullptr, NB, s);
    } else {
        launch_scan_dir<false, false>(grid, wsB, elemsB, wsA, elemsA, nullptr, nullptr, NB, s);
    }
    return hipGetLastError();
}

// ============================================================================ partial sums
// out[b][h][t][d] = sum over bucket tiles st of part[st * tile + ((b * H + h) * T + t) * D + d].
// Fast form: grid (chunks of one (b, h) slab, B*H), 32-bit index math, V = 4 consecutive head-dim
// elements per thread with 16-byte loads and 16-/8-byte stores. The general form (one element per
// thread, 64-bit index math) serves shapes the fast form does not fit.
template <int V>
__global__ __launch_bounds__(256) void race_reduce_partials_vec(const float *part, int n_st, int64_t tile,
                                                                OutView out, int H, int T, int D)
{
    const int bh = blockIdx.y, b = bh / H, h = bh % H;
    const int DV = D / V;
    const int j = blockIdx.x * 256 + threadIdx.x;  // (t, group of V head-dim elements) within the slab
    if (j >= T * DV)
        return;
    const int t = j / DV, d = (j - t * DV) * V;
    const float *src = part + ((int64_t)bh * T + t) * D + d;
    f32x4 acc = *reinterpret_cast<const f32x4 *>(src);
    for (int st = 1; st < n_st; ++st) {
        const f32x4 x = *reinterpret_cast<const f32x4 *>(src + (int64_t)st * tile);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            acc[e] += x[e];
    }
    const int64_t off = b * out.sb + h * out.sh + (int64_t)t * out.st + d;
    if (out.f32) {
        *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(out.p) + off) = acc;
    } else {
        bf16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w[e] = (__bf16)acc[e];
        *reinterpret_cast<bf16x4 *>(reinterpret_cast<__bf16 *>(out.p) + off) = w;
    }
}

__global__ void race_reduce_partials_any(const float *part, int n_st, int64_t tile, OutView out, int H,
                                         int T, int D, int64_t total)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total)
        return;
    float acc = 0.0f;
    for (int st = 0; st < n_st; ++st)
        acc += part[(int64_t)st * tile + i];
    const int d = (int)(i % D);
    const int64_t r = i / D;
    const int t = (int)(r % T);
    const int64_t bh = r / T;
    const int h = (int)(bh % H);
    const int64_t b = bh / H;
    const int64_t off = b * out.sb + h * out.sh + (int64_t)t * out.st + d;
    if (out.f32)
        reinterpret_cast<float *>(out.p)[off] = acc;
    else
        reinterpret_cast<__bf16 *>(out.p)[off] = (__bf16)acc;
}

hipError_t launch_reduce_partials(const float *part, int n_st, int64_t tile, const OutView &out,
                                  int B, int H, int T, int D, hipStream_t s)
{
    const int64_t total = (int64_t)B * H * T * D;
    const int esz = out.f32 ? 4 : 2;
    const bool vec = D % 4 == 0 && out.sb % 4 == 0 && out.sh % 4 == 0 && out.st % 4 == 0 && tile % 4 == 0 &&
                     reinterpret_cast<uintptr_t>(part) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(out.p) % (4 * esz) == 0 && (int64_t)T * (D / 4) < (1LL << 31) - 256 &&
                     (int64_t)B * H <= 65535;
    if (vec) {
        const int64_t per_slab = (int64_t)T * (D / 4);
        hipLaunchKernelGGL(race_reduce_partials_vec<4>, dim3((unsigned)((per_slab + 255) / 256), (unsigned)(B * H)),
                           dim3(256), 0, s, part, n_st, tile, out, H, T, D);
    } else {
        hipLaunchKernelGGL(race_reduce_partials_any, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                           part, n_st, tile, out, H, T, D, total);
    }
    return hipGetLastError();
}

// ============================================================================ soft-hash
// Per table: p[r] = prod_k (bit_k(r) ? s1_k : s0_k), s1 = sigmoid(2u), s0 = sigmoid(-2u), with
// bit k = 0 the most significant bit of r (corner order of itertools.product([-1, 1])). The
// kernels are compiled per bit count KB = 1..8, so every per-table array stays in registers;
// for KB <= 4 all 2^KB probabilities are expanded in registers and the backward's corner sums
// run as a butterfly over the bits.
RACE_DEV void sigm_pair(float u, float &s0, float &s1)
{
    const float e = __expf(-2.0f * sig_arg(u));
    s1 = frcp(1.0f + e);
    s0 = e * s1;
}

template <int KB>
RACE_DEV float corner_prob(const float *s0, const float *s1, int r)
{
    float p = 1.0f;
#pragma unroll
    for (int k = 0; k < KB; ++k)
        p *= ((r >> (KB - 1 - k)) & 1) ? s1[k] : s0[k];
    return p;
}

// all 2^KB corner probabilities; each factor enters as the lowest index bit and is shifted up
// by the later ones, so factor 0 ends as the most significant bit
template <int KB>
RACE_DEV void corner_probs(const float *s0, const float *s1, float *p)
{
    p[0] = 1.0f;
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        const int n = 1 << k;
#pragma unroll
        for (int i = n - 1; i >= 0; --i) {
            const float pi = p[i];
            p[2 * i + 1] = pi * s1[k];
            p[2 * i] = pi * s0[k];
        }
    }
}

// LDS of one soft-hash workgroup (floats):
//   sPl [DX][PL]  planes of one member, zero beyond (D, LK); PL is 4 x odd words, so 16-byte reads by
//                 16 lanes of consecutive rows d cover the 64 banks once
//   sX  [TT][DX]  input rows, zero beyond D (DX = D rounded up to 4)
//   sU  [TT][LK]  tanh(projection) / scale
//   sGP [TT][PG]  backward only: d loss / d projection, zero beyond LK (PG = LK rounded up to 4)
__host__ __device__ inline int sh_dx(int D) { return (D + 3) & ~3; }
__host__ __device__ inline int sh_pg(int LK) { return (LK + 3) & ~3; }
__host__ __device__ inline int sh_pl(int LK) { return sh_pg(LK) + ((sh_pg(LK) & 4) ? 0 : 4); }
constexpr int SH_RB = 4;  // rows per thread in the two LDS products

RACE_DEV void sh_load_planes(float *sPl, const float *planes, const SoftHashParams &P)
{
    const int DX = sh_dx(P.D), PL = sh_pl(P.LK);
    for (int i = threadIdx.x; i < DX * PL; i += 256) {
        const int d = i / PL, j = i - d * PL;
        float v = 0.0f;
        if (d < P.D && j < P.LK) {
            v = planes[d * P.LK + j];
            if (P.round_planes)
                v = (float)(__bf16)v;
        }
        sPl[i] = v;
    }
}

// The logits divisor: the device scalar when one is given (a learnable temperature that stays in
// device memory, so its caller never reads it back to the host), else the launch argument.
RACE_DEV float sh_scale(const SoftHashParams &P) { return P.scale_dev ? *P.scale_dev : P.scale; }
RACE_DEV float sh_inv_scale(const SoftHashParams &P) { return P.scale_dev ? 1.0f / *P.scale_dev : P.inv_scale; }

// x rows of one tile into sX. vec: D % 4 == 0, and every row starts at a multiple of 4 elements
// of a buffer aligned to 4 elements, so a row is read as runs of 4 elements (16 or 8 bytes)
template <class TX>
RACE_DEV void sh_load_x(float *sX, const SoftHashParams &P, int b, int h, int t0, int nv, bool vec)
{
    const int DX = sh_dx(P.D);
    const TX *x = reinterpret_cast<const TX *>(P.x.p);
    if (vec) {
        typedef TX tx4 __attribute__((ext_vector_type(4)));
        const int D4 = DX / 4;
        for (int i = threadIdx.x; i < SH_TT * D4; i += 256) {
            const int r = i / D4, d = (i - r * D4) * 4;
            f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
            if (r < nv) {
                const tx4 w = *reinterpret_cast<const tx4 *>(x + b * P.x.sb + h * P.x.sh + (int64_t)(t0 + r) * P.x.st + d);
                v = f32x4{(float)w[0], (float)w[1], (float)w[2], (float)w[3]};
            }
            *reinterpret_cast<f32x4 *>(sX + r * DX + d) = v;
        }
        return;
    }
    for (int i = threadIdx.x; i < SH_TT * DX; i += 256) {
        const int r = i / DX, d = i - r * DX;
        sX[i] = (r < nv && d < P.D) ? (float)x[b * P.x.sb + h * P.x.sh + (int64_t)(t0 + r) * P.x.st + d] : 0.0f;
    }
}

template <class TX>
RACE_DEV bool sh_x_vec(const SoftHashParams &P)
{
    return (P.D & 3) == 0 && (reinterpret_cast<uintptr_t>(P.x.p) & (4 * sizeof(TX) - 1)) == 0 && (P.x.sb & 3) == 0 &&
           (P.x.sh & 3) == 0 && (P.x.st & 3) == 0;
}

// sU[r][j] = tanh(sum_d x[r][d] planes[d][j]) / scale. A thread owns SH_RB rows of one column j:
// x is read as 16-byte runs that all lanes of a row group share, planes as one word per row d
RACE_DEV void sh_project(const float *sX, const float *sPl, float *sU, const SoftHashParams &P)
{
    const int DX = sh_dx(P.D), PL = sh_pl(P.LK), LK = P.LK;
    for (int i = threadIdx.x; i < (SH_TT / SH_RB) * LK; i += 256) {
        const int rg = i / LK, j = i - rg * LK;
        const float *xr = sX + rg * SH_RB * DX;
        float acc[SH_RB] = {};
        for (int d = 0; d < DX; d += 4) {
            float pl[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                pl[e] = sPl[(d + e) * PL + j];
#pragma unroll
            for (int q = 0; q < SH_RB; ++q) {
                const f32x4 xv = *reinterpret_cast<const f32x4 *>(xr + q * DX + d);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[q] += xv[e] * pl[e];
            }
        }
#pragma unroll
        for (int q = 0; q < SH_RB; ++q)
            sU[(rg * SH_RB + q) * LK + j] = tanh_f(acc[q]) * sh_inv_scale(P);
    }
}

template <class TX, int KB>
__global__ __launch_bounds__(256) void race_softhash_fwd(SoftHashParams P)
{
    extern __shared__ float sm[];
    const int DX = sh_dx(P.D);
    float *sPl = sm;
    float *sX = sPl + DX * sh_pl(P.LK);
    float *sU = sX + SH_TT * DX;
    const int bh = blockIdx.y;
    const int m = blockIdx.z;            // ensemble member (unshared planes) or 0
    const int b = bh / P.H, h = bh % P.H;
    const int ntt = (P.T + SH_TT - 1) / SH_TT;
    const int tt1 = min(ntt, ((int)blockIdx.x + 1) * P.tpw);
    constexpr int R = 1 << KB;
    const int S = P.L * R;
    float *out = P.probs + ((int64_t)m * P.B * P.H + bh) * P.T * S;
    // every token's run of R corners starts 16-byte aligned when the buffer does and R % 4 == 0
    const bool vec_out = (reinterpret_cast<uintptr_t>(P.probs) & 15) == 0;
    const bool vec_x = sh_x_vec<TX>(P);
    sh_load_planes(sPl, P.planes + (int64_t)m * P.plane_stride, P);
    // tiles of SH_TT tokens; sX is free again once the projection's barrier is passed, and the
    // barrier after the x load keeps the next projection from overwriting sU under the readers
    for (int tt = blockIdx.x * P.tpw; tt < tt1; ++tt) {
        const int t0 = tt * SH_TT;
        const int nv = min(SH_TT, P.T - t0);
        sh_load_x<TX>(sX, P, b, h, t0, nv, vec_x);
        __syncthreads();
        sh_project(sX, sPl, sU, P);
        __syncthreads();
        if constexpr (KB >= 2 && KB <= 4) {
            if (vec_out) {
                // R / 4 threads per (token, table), each storing 4 consecutive corners: consecutive
                // threads write consecutive 16-byte runs. Corner c = 4q + c2 takes its KB - 2 high
                // bits from q; products in the same order as corner_probs (bitwise equal).
                constexpr int Q = R / 4;
                for (int i = threadIdx.x; i < nv * P.L * Q; i += blockDim.x) {
                    const int it = i / Q, q = i - it * Q;
                    const int r = it / P.L, l = it - r * P.L;
                    float s0[KB], s1[KB];
#pragma unroll
                    for (int k = 0; k < KB; ++k)
                        sigm_pair(sU[r * P.LK + l * KB + k], s0[k], s1[k]);
                    float pre = 1.0f;
#pragma unroll
                    for (int k = 0; k < KB - 2; ++k)
                        pre *= ((q >> (KB - 3 - k)) & 1) ? s1[k] : s0[k];
                    const float a0 = pre * s0[KB - 2], a1 = pre * s1[KB - 2];
                    *reinterpret_cast<f32x4 *>(out + (int64_t)(t0 + r) * S + l * R + 4 * q) =
                        f32x4{a0 * s0[KB - 1], a0 * s1[KB - 1], a1 * s0[KB - 1], a1 * s1[KB - 1]};
                }
                continue;
            }
        }
        for (int i = threadIdx.x; i < nv * P.L; i += blockDim.x) {
            const int r = i / P.L, l = i % P.L;
            float s0[KB], s1[KB];
#pragma unroll
            for (int k = 0; k < KB; ++k)
                sigm_pair(sU[r * P.LK + l * KB + k], s0[k], s1[k]);
            float *o = out + (int64_t)(t0 + r) * S + l * R;
            if constexpr (KB <= 4) {
                float p[R];
                corner_probs<KB>(s0, s1, p);
#pragma unroll
                for (int c = 0; c < R; ++c)
                    o[c] = p[c];
            } else {
                for (int c = 0; c < R; ++c)
                    o[c] = corner_prob<KB>(s0, s1, c);
            }
        }
    }
}

// dx[b,h,t,:] = sum_m sum_j gproj_m[t,j] planes_m[:, j]. DI: dx items per thread (D <= 32 * DI),
// so the accumulators held across a tile take no more registers than the head dim needs
template <class TX, int KB, int DI>
__global__ __launch_bounds__(256) void race_softhash_bwd(SoftHashParams P)
{
    extern __shared__ float sm[];
    const int DX = sh_dx(P.D), PL = sh_pl(P.LK), PG = sh_pg(P.LK);
    float *sPl = sm;
    float *sX = sPl + DX * PL;
    float *sU = sX + SH_TT * DX;
    float *sGP = sU + SH_TT * P.LK;
    const int bh = blockIdx.y;
    const int b = bh / P.H, h = bh % P.H;
    const int ntt = (P.T + SH_TT - 1) / SH_TT;
    const int tt1 = min(ntt, ((int)blockIdx.x + 1) * P.tpw);
    for (int i = threadIdx.x; i < SH_TT * PG; i += 256)  // the padding columns stay zero
        sGP[i] = 0.0f;
    if (P.M == 1)  // one set of planes for every tile
        sh_load_planes(sPl, P.planes, P);
    constexpr int R = 1 << KB;
    const int S = P.L * R;
    const bool vec_in = (reinterpret_cast<uintptr_t>(P.gprobs) & 15) == 0;
    const bool vec_x = sh_x_vec<TX>(P);
    // dx items: (row group, d) pairs, SH_RB rows each: SH_TT / SH_RB * D of them over 256 threads
    constexpr int MAXI = DI;
    static_assert(SH_TT / SH_RB * 32 == 256, "D <= 32 * DI gives at most DI items per thread");
    float gsu = 0.0f;  // sum of gu * u over this thread's (token, table) items
    // tiles of SH_TT tokens. Per member: barrier, planes (several members only), barrier,
    // projection, barrier, gproj, barrier, dx products; every LDS buffer is rewritten only after
    // a barrier that all of its readers have passed
    for (int tt = blockIdx.x * P.tpw; tt < tt1; ++tt) {
        const int t0 = tt * SH_TT;
        const int nv = min(SH_TT, P.T - t0);
        float gx[MAXI][SH_RB];
#pragma unroll
        for (int o = 0; o < MAXI; ++o)
#pragma unroll
            for (int q = 0; q < SH_RB; ++q)
                gx[o][q] = 0.0f;
        sh_load_x<TX>(sX, P, b, h, t0, nv, vec_x);
        for (int m = 0; m < P.M; ++m) {
            __syncthreads();
            if (P.M > 1) {
                sh_load_planes(sPl, P.planes + (int64_t)(P.unshared ? m : 0) * P.plane_stride, P);
                __syncthreads();
            }
            sh_project(sX, sPl, sU, P);
            __syncthreads();
            const float *gprobs = P.gprobs + ((int64_t)m * P.B * P.H + bh) * P.T * S;
            for (int i = threadIdx.x; i < SH_TT * P.L; i += blockDim.x) {
                const int r = i / P.L, l = i % P.L;
                float u[KB], s0[KB], s1[KB], gu[KB];
#pragma unroll
                for (int k = 0; k < KB; ++k) {
                    u[k] = sU[r * P.LK + l * KB + k];
                    sigm_pair(u[k], s0[k], s1[k]);
                    gu[k] = 0.0f;
                }
                if (r < nv) {
                    const float *gp = gprobs + (int64_t)(t0 + r) * S + l * R;
                    if constexpr (KB <= 4) {
                        // gz_c = p_c (gp_c - sum p gp); gu_k = sum_c sign_k(c) gz_c with sign +1 where
                        // bit k of c is set: a butterfly from the least significant bit, pair sums
                        // feed the next level and pair differences sum to that bit's gu
                        float p[R], z[R], g[R];
                        if (R % 4 == 0 && vec_in) {
#pragma unroll
                            for (int c = 0; c < R; c += 4) {
                                const f32x4 w = *reinterpret_cast<const f32x4 *>(gp + c);
                                g[c] = w[0];
                                g[c + 1] = w[1];
                                g[c + 2] = w[2];
                                g[c + 3] = w[3];
                            }
                        } else {
#pragma unroll
                            for (int c = 0; c < R; ++c)
                                g[c] = gp[c];
                        }
                        corner_probs<KB>(s0, s1, p);
                        float dot = 0.0f;
#pragma unroll
                        for (int c = 0; c < R; ++c)
                            dot += p[c] * g[c];
#pragma unroll
                        for (int c = 0; c < R; ++c)
                            z[c] = p[c] * (g[c] - dot);
#pragma unroll
                        for (int lvl = 0; lvl < KB; ++lvl) {
                            const int n = R >> (lvl + 1);
                            float acc = 0.0f;
#pragma unroll
                            for (int q = 0; q < n; ++q) {
                                acc += z[2 * q + 1] - z[2 * q];
                                z[q] = z[2 * q] + z[2 * q + 1];
                            }
                            gu[KB - 1 - lvl] = acc;
                        }
                    } else {
                        float dot = 0.0f;
                        for (int c = 0; c < R; ++c)
                            dot += corner_prob<KB>(s0, s1, c) * gp[c];
                        for (int c = 0; c < R; ++c) {
                            const float gz = corner_prob<KB>(s0, s1, c) * (gp[c] - dot);
#pragma unroll
                            for (int k = 0; k < KB; ++k)
                                gu[k] += ((c >> (KB - 1 - k)) & 1) ? gz : -gz;
                        }
                    }
#pragma unroll
                    for (int k = 0; k < KB; ++k)
                        gsu += gu[k] * u[k];
                }
#pragma unroll
                for (int k = 0; k < KB; ++k) {
                    const float th = u[k] * sh_scale(P);
                    sGP[r * PG + l * KB + k] = gu[k] * sh_inv_scale(P) * (1.0f - th * th);
                }
            }
            __syncthreads();
            // gx[r][d] += sum_j gproj[r][j] planes[d][j]: SH_RB rows of one d per item, both operands
            // read as 16-byte runs over j (gproj shared by the lanes of a row group)
#pragma unroll
            for (int o = 0; o < MAXI; ++o) {
                const int i = threadIdx.x + o * 256;
                if (i < (SH_TT / SH_RB) * P.D) {
                    const int rg = i / P.D, d = i - rg * P.D;
                    const float *gr = sGP + rg * SH_RB * PG;
                    const float *pr = sPl + d * PL;
                    float acc[SH_RB] = {};
                    for (int j = 0; j < PG; j += 4) {
                        const f32x4 pv = *reinterpret_cast<const f32x4 *>(pr + j);
#pragma unroll
                        for (int q = 0; q < SH_RB; ++q) {
                            const f32x4 gv = *reinterpret_cast<const f32x4 *>(gr + q * PG + j);
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                acc[q] += gv[e] * pv[e];
                        }
                    }
#pragma unroll
                    for (int q = 0; q < SH_RB; ++q)
                        gx[o][q] += acc[q];
                }
            }
        }
        TX *dx = reinterpret_cast<TX *>(const_cast<void *>(P.dx.p));
#pragma unroll
        for (int o = 0; o < MAXI; ++o) {
            const int i = threadIdx.x + o * 256;
            if (i < (SH_TT / SH_RB) * P.D) {
                const int rg = i / P.D, d = i - rg * P.D;
#pragma unroll
                for (int q = 0; q < SH_RB; ++q) {
                    const int r = rg * SH_RB + q;
                    if (r < nv)
                        dx[b * P.dx.sb + h * P.dx.sh + (int64_t)(t0 + r) * P.dx.st + d] = (TX)gx[o][q];
                }
            }
        }
    }
    if (P.gscale) {
        // workgroup sum of gu * u: d loss / d scale = -(1/scale) * (sum over all workgroups)
        __shared__ float red[4];
        for (int o = 32; o > 0; o >>= 1)
            gsu += __shfl_xor(gsu, o);
        if ((threadIdx.x & 63) == 0)
            red[threadIdx.x >> 6] = gsu;
        __syncthreads();
        if (threadIdx.x == 0)
            P.gscale[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = red[0] + red[1] + red[2] + red[3];
    }
}

// ---------------------------------------------------------------------------- soft-hash on MFMA
// Soft-hash for L*K <= 32 and K <= 4 on fp32 MFMA (v_mfma_f32_16x16x4_f32), one 16-token tile per
// wave and no workgroup barrier after the planes are loaded. Lane (n = lane % 16, g = lane / 16)
// loads its token's x at d = 16 jj + 4 g .. + 3 (one 16-byte or 8-byte run per jj, straight from
// HBM), which is the K index of k-steps (jj, e) of the projection
//   u^T[j][t] = sum_d planes^T[j][d] x[t][d]   (M = plane, N = token, K = d)
// whose A fragment reads planes^T rows as 16-byte runs (pitch an odd multiple of 8 words:
// conflict-free). The backward's
//   dx^T[d][t] = sum_j planes[d][j] gproj[t][j]   (M = d, N = token, K = plane)
// leaves four consecutive d of one token in a lane, stored as one run. u and gproj pass through
// per-wave LDS rows between the MFMA layout and the (token, table) items.
constexpr int SHM_W = 4;  // waves per workgroup

// compiled head-dim class of the matrix-core soft-hash kernels
__host__ __device__ inline int shm_dp(int D) { return D <= 64 ? 64 : D <= 128 ? 128 : 256; }

struct ShmLayout {
    int DX16, PT, PD, PU, njt;  // d rounded to the head-dim class, pitches (floats), plane tiles of 16
    __host__ __device__ ShmLayout(int D, int LK)
    {
        DX16 = shm_dp(D);
        PT = DX16 + 8;  // odd multiple of 8
        PD = (LK + 3) & ~3;
        if (((PD / 4) & 1) == 0)
            PD += 4;  // 4 x odd
        njt = (LK + 15) / 16;
        PU = njt == 1 ? 24 : 40;  // odd multiple of 8, >= 16 njt
    }
    // floats: planes^T [16 njt][PT], per-wave u [SHM_W][16][PU]; backward also planes [DX16][PD] and
    // per-wave gproj [SHM_W][16][PD]; then, for the 128 and 256 classes (whose x and dx rows move
    // through it), per-wave row staging [SHM_W][16][SHS_LD] at stage_off
    static constexpr int SHS_LD = 32 + 4;
    __host__ __device__ int stage_off(bool bwd) const
    {
        return 16 * njt * PT + SHM_W * 16 * PU + (bwd ? DX16 * PD + SHM_W * 16 * PD : 0);
    }
    __host__ __device__ int floats(bool bwd) const
    {
        return stage_off(bwd) + (DX16 >= 128 ? SHM_W * 16 * SHS_LD : 0);
    }
};

bool softhash_mfma_ok(int D, int L, int K, int M, int bwd)
{
    return D <= 256 && L * K <= 32 && K <= 4 && (!bwd || M == 1);
}

// planes of one member into sPlT [16 njt][PT] (and sPl [DX16][PD]), zero beyond (LK, D)
RACE_DEV void shm_load_planes(float *sPlT, float *sPl, const float *planes, const SoftHashParams &P,
                              const ShmLayout &Y)
{
    for (int i = threadIdx.x; i < 16 * Y.njt * Y.DX16; i += SHM_W * 64) {
        const int j = i / Y.DX16, d = i - j * Y.DX16;
        float v = 0.0f;
        if (d < P.D && j < P.LK) {
            v = planes[d * P.LK + j];
            if (P.round_planes)
                v = (float)(__bf16)v;
        }
        sPlT[j * Y.PT + d] = v;
        if (sPl && j < Y.PD)
            sPl[d * Y.PD + j] = v;
    }
    if (sPl) {  // columns 16 njt .. PD (PD can exceed the plane tiles by 4)
        for (int i = threadIdx.x; i < Y.DX16 * Y.PD; i += SHM_W * 64) {
            const int d = i / Y.PD, j = i - d * Y.PD;
            if (j >= 16 * Y.njt)
                sPl[i] = 0.0f;
        }
    }
}

// u = tanh(x . planes) / scale of this wave's 16 tokens t0 .. t0 + 15 (those < tok1) into its sU
// rows [16][PU]. x moves in row-contiguous runs: lane l loads row it * 8 + l / 8 (it = 0, 1) at
// columns 32 c + 4 (l % 8) of each 32-column chunk c (8 rows x 4 elements per lane and row), the
// chunk passes through the wave's staging rows sX [16][SHS_LD] (pitch 4 x odd words), and lane
// (n, g) reads back columns 16 j + 4 g .. + 3 of row n, the K index of k-steps (j, e) of
//   u^T[j][t] = sum_d planes^T[j][d] x[t][d]   (M = plane, N = token, K = d)
template <class TX, int NJT, int DP>
RACE_DEV void shm_project(float *sU, float *sX, const float *sPlT, const SoftHashParams &P, const ShmLayout &Y,
                          const TX *x, int t0, int tok1, bool vec, int lane, int n16, int g)
{
    constexpr int NJ = DP / 16, LD = ShmLayout::SHS_LD;
    f32x4 acc[NJT];
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt)
        acc[jt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (DP < 128) {
        // 64-column rows: lane (n, g) loads its own row's columns 16 j + 4 g .. + 3 straight into the
        // fragments (clamped addresses, masked lanes selected to zero; measured faster than staging)
        const int t = min(t0 + n16, tok1 - 1);
        const bool ok = t0 + n16 < tok1;
        const TX *xrow = x + (int64_t)t * P.x.st;
        f32x4 xv[NJ];
        if (vec) {
            typedef TX tx4 __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int d = 16 * j + 4 * g;
                const tx4 w = *reinterpret_cast<const tx4 *>(xrow + min(d, P.D - 4));
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    xv[j][e] = ok && d < P.D ? (float)w[e] : 0.0f;
            }
        } else {
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int d = 16 * j + 4 * g + e;
                    const float v = (float)xrow[min(d, P.D - 1)];
                    xv[j][e] = ok && d < P.D ? v : 0.0f;
                }
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int jt = 0; jt < NJT; ++jt) {
                const f32x4 pt = *reinterpret_cast<const f32x4 *>(sPlT + (16 * jt + n16) * Y.PT + 16 * j + 4 * g);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    EngF32::mma(acc[jt], pt[e], xv[j][e]);
            }
    } else {
        f32x4 xr[DP / 32][2];
#pragma unroll
        for (int c = 0; c < DP / 32; ++c)
#pragma unroll
            for (int it = 0; it < 2; ++it) {
                const int r = it * 8 + lane / 8, col = 32 * c + 4 * (lane % 8);
                f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
                if (t0 + r < tok1 && col < P.D) {
                    const TX *p = x + (int64_t)(t0 + r) * P.x.st + col;
                    if (vec) {
                        typedef TX tx4 __attribute__((ext_vector_type(4)));
                        const tx4 w = *reinterpret_cast<const tx4 *>(p);
                        v = f32x4{(float)w[0], (float)w[1], (float)w[2], (float)w[3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            v[e] = col + e < P.D ? (float)p[e] : 0.0f;
                    }
                }
                xr[c][it] = v;
            }
#pragma unroll
        for (int c = 0; c < DP / 32; ++c) {
#pragma unroll
            for (int it = 0; it < 2; ++it)
                *reinterpret_cast<f32x4 *>(sX + (it * 8 + lane / 8) * LD + 4 * (lane % 8)) = xr[c][it];
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const f32x4 xv = *reinterpret_cast<const f32x4 *>(sX + n16 * LD + 16 * jj + 4 * g);
                const int j = 2 * c + jj;
#pragma unroll
                for (int jt = 0; jt < NJT; ++jt) {
                    const f32x4 pt = *reinterpret_cast<const f32x4 *>(sPlT + (16 * jt + n16) * Y.PT + 16 * j + 4 * g);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        EngF32::mma(acc[jt], pt[e], xv[e]);
                }
            }
        }
    }
    static_assert(NJ == 2 * (DP / 32), "32-column chunks of two 16-wide k runs");
    // accumulator rows: planes 16 jt + 4 g + e of token n16
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt) {
        f32x4 u;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            u[e] = tanh_f(acc[jt][e]) * sh_inv_scale(P);
        *reinterpret_cast<f32x4 *>(sU + n16 * Y.PU + 16 * jt + 4 * g) = u;
    }
}

template <class TX, int KB, int NJT, int DP>
__global__ __launch_bounds__(SHM_W * 64) void race_softhash_fwd_mfma(SoftHashParams P)
{
    extern __shared__ float sm[];
    const ShmLayout Y(P.D, P.LK);
    float *sPlT = sm;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, n16 = lane & 15, g = lane >> 4;
    float *sU = sPlT + 16 * NJT * Y.PT + w * 16 * Y.PU;
    float *sX = sm + Y.stage_off(false) + w * 16 * ShmLayout::SHS_LD;
    const int bh = blockIdx.y, m = blockIdx.z;
    const int b = bh / P.H, h = bh % P.H;
    constexpr int R = 1 << KB;
    const int S = P.L * R;
    float *out = P.probs + ((int64_t)m * P.B * P.H + bh) * P.T * S;
    const bool vec_out = (reinterpret_cast<uintptr_t>(P.probs) & 15) == 0;
    const bool vec_x = sh_x_vec<TX>(P);
    const TX *x = reinterpret_cast<const TX *>(P.x.p) + b * P.x.sb + h * P.x.sh;
    shm_load_planes(sPlT, nullptr, P.planes + (int64_t)m * P.plane_stride, P, Y);
    __syncthreads();
    const int span = P.tpw * SHM_W * 16;
    const int tok0 = blockIdx.x * span, tok1 = min(P.T, tok0 + span);
    for (int t0 = tok0 + 16 * w; t0 < tok1; t0 += 16 * SHM_W) {
        shm_project<TX, NJT, DP>(sU, sX, sPlT, P, Y, x, t0, tok1, vec_x, lane, n16, g);
        const int nv = min(16, tok1 - t0);
        if constexpr (KB >= 2) {
            if (vec_out) {
                // R / 4 lanes per (token, table), each storing 4 consecutive corners: consecutive
                // lanes write consecutive 16-byte runs. Corner c = 4q + c2 takes its KB - 2 high bits
                // from q; products in the same order as corner_probs
                constexpr int Q = R / 4;
                for (int i = lane; i < nv * P.L * Q; i += 64) {
                    const int it = i / Q, q = i - it * Q;
                    const int r = it / P.L, l = it - r * P.L;
                    float s0[KB], s1[KB];
#pragma unroll
                    for (int k = 0; k < KB; ++k)
                        sigm_pair(sU[r * Y.PU + l * KB + k], s0[k], s1[k]);
                    float pre = 1.0f;
#pragma unroll
                    for (int k = 0; k < KB - 2; ++k)
                        pre *= ((q >> (KB - 3 - k)) & 1) ? s1[k] : s0[k];
                    const float a0 = pre * s0[KB - 2], a1 = pre * s1[KB - 2];
                    *reinterpret_cast<f32x4 *>(out + (int64_t)(t0 + r) * S + l * R + 4 * q) =
                        f32x4{a0 * s0[KB - 1], a0 * s1[KB - 1], a1 * s0[KB - 1], a1 * s1[KB - 1]};
                }
                continue;
            }
        }
        for (int i = lane; i < nv * P.L; i += 64) {
            const int r = i / P.L, l = i - r * P.L;
            float s0[KB], s1[KB], p[R];
#pragma unroll
            for (int k = 0; k < KB; ++k)
                sigm_pair(sU[r * Y.PU + l * KB + k], s0[k], s1[k]);
            corner_probs<KB>(s0, s1, p);
            float *o = out + (int64_t)(t0 + r) * S + l * R;
#pragma unroll
            for (int c = 0; c < R; ++c)
                o[c] = p[c];
        }
    }
}

template <class TX, int KB, int NJT, int DP>
__global__ __launch_bounds__(SHM_W * 64) void race_softhash_bwd_mfma(SoftHashParams P)
{
    extern __shared__ float sm[];
    const ShmLayout Y(P.D, P.LK);
    float *sPlT = sm;
    float *sPl = sPlT + 16 * NJT * Y.PT;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, n16 = lane & 15, g = lane >> 4;
    float *sU = sPl + Y.DX16 * Y.PD + w * 16 * Y.PU;
    float *sGP = sPl + Y.DX16 * Y.PD + SHM_W * 16 * Y.PU + w * 16 * Y.PD;
    float *sX = sm + Y.stage_off(true) + w * 16 * ShmLayout::SHS_LD;
    const int bh = blockIdx.y;
    const int b = bh / P.H, h = bh % P.H;
    constexpr int R = 1 << KB;
    const int S = P.L * R;
    const bool vec_in = (reinterpret_cast<uintptr_t>(P.gprobs) & 15) == 0;
    const bool vec_x = sh_x_vec<TX>(P);
    const bool vec_dx = (P.D & 3) == 0 && (reinterpret_cast<uintptr_t>(P.dx.p) & (4 * sizeof(TX) - 1)) == 0 &&
                        (P.dx.sb & 3) == 0 && (P.dx.sh & 3) == 0 && (P.dx.st & 3) == 0;
    const TX *x = reinterpret_cast<const TX *>(P.x.p) + b * P.x.sb + h * P.x.sh;
    TX *dx = reinterpret_cast<TX *>(const_cast<void *>(P.dx.p)) + b * P.dx.sb + h * P.dx.sh;
    const float *gprobs = P.gprobs + (int64_t)bh * P.T * S;
    for (int i = lane; i < 16 * Y.PD; i += 64)  // columns >= L*K stay zero
        sGP[i] = 0.0f;
    shm_load_planes(sPlT, sPl, P.planes, P, Y);
    __syncthreads();
    float gsu = 0.0f;  // sum of gu * u over this lane's (token, table) items
    const int span = P.tpw * SHM_W * 16;
    const int tok0 = blockIdx.x * span, tok1 = min(P.T, tok0 + span);
    for (int t0 = tok0 + 16 * w; t0 < tok1; t0 += 16 * SHM_W) {
        shm_project<TX, NJT, DP>(sU, sX, sPlT, P, Y, x, t0, tok1, vec_x, lane, n16, g);
        // (token, table) items: gu_k = d loss / d u_k, gproj = gu * (1 - tanh^2) / scale
        for (int i = lane; i < 16 * P.L; i += 64) {
            const int r = i / P.L, l = i - r * P.L;
            float u[KB], s0[KB], s1[KB], gu[KB];
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                u[k] = sU[r * Y.PU + l * KB + k];
                sigm_pair(u[k], s0[k], s1[k]);
                gu[k] = 0.0f;
            }
            if (t0 + r < tok1) {
                const float *gp = gprobs + (int64_t)(t0 + r) * S + l * R;
                // gz_c = p_c (gp_c - sum p gp); gu_k = sum_c sign_k(c) gz_c with sign +1 where bit k
                // of c is set: a butterfly from the least significant bit
                float p[R], z[R], gr[R];
                if (R % 4 == 0 && vec_in) {
#pragma unroll
                    for (int c = 0; c < R; c += 4) {
                        const f32x4 v4 = *reinterpret_cast<const f32x4 *>(gp + c);
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            gr[c + e] = v4[e];
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < R; ++c)
                        gr[c] = gp[c];
                }
                corner_probs<KB>(s0, s1, p);
                float dot = 0.0f;
#pragma unroll
                for (int c = 0; c < R; ++c)
                    dot += p[c] * gr[c];
#pragma unroll
                for (int c = 0; c < R; ++c)
                    z[c] = p[c] * (gr[c] - dot);
#pragma unroll
                for (int lvl = 0; lvl < KB; ++lvl) {
                    const int n = R >> (lvl + 1);
                    float acc = 0.0f;
#pragma unroll
                    for (int q = 0; q < n; ++q) {
                        acc += z[2 * q + 1] - z[2 * q];
                        z[q] = z[2 * q] + z[2 * q + 1];
                    }
                    gu[KB - 1 - lvl] = acc;
                }
#pragma unroll
                for (int k = 0; k < KB; ++k)
                    gsu += gu[k] * u[k];
            }
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                const float th = u[k] * sh_scale(P);
                sGP[r * Y.PD + l * KB + k] = gu[k] * sh_inv_scale(P) * (1.0f - th * th);
            }
        }
        // dx^T tiles of 16 d: A = planes rows d (4-byte reads, pitch 4 x odd), B = gproj of token n16;
        // k-steps over the planes (L*K <= 16 NJT, rounded to 4). Two tiles (32 columns) at a time pass
        // through the staging rows and leave as row-contiguous runs (8 rows per store instruction)
        const int nks = (P.LK + 3) / 4;
        constexpr int LD = ShmLayout::SHS_LD;
        if constexpr (DP < 128) {
            // 64-column rows: each lane stores its own row's four columns per tile (measured faster)
            const int t = t0 + n16;
            TX *o = dx + (int64_t)t * P.dx.st;
#pragma unroll
            for (int j = 0; j < DP / 16; ++j) {
                f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
                for (int kk = 0; kk < nks; ++kk)
                    EngF32::mma(acc, sPl[(16 * j + n16) * Y.PD + 4 * kk + g], sGP[n16 * Y.PD + 4 * kk + g]);
                const int d = 16 * j + 4 * g;
                if (t < tok1 && d < P.D) {
                    if (vec_dx) {
                        typedef TX tx4 __attribute__((ext_vector_type(4)));
                        *reinterpret_cast<tx4 *>(o + d) = tx4{(TX)acc[0], (TX)acc[1], (TX)acc[2], (TX)acc[3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (d + e < P.D)
                                o[d + e] = (TX)acc[e];
                    }
                }
            }
            continue;
        }
#pragma unroll
        for (int c = 0; c < DP / 32; ++c) {
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int j = 2 * c + jj;
                f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
                for (int kk = 0; kk < nks; ++kk)
                    EngF32::mma(acc, sPl[(16 * j + n16) * Y.PD + 4 * kk + g], sGP[n16 * Y.PD + 4 * kk + g]);
                *reinterpret_cast<f32x4 *>(sX + n16 * LD + 16 * jj + 4 * g) = acc;
            }
#pragma unroll
            for (int it = 0; it < 2; ++it) {
                const int r = it * 8 + lane / 8, cl = 4 * (lane % 8), d = 32 * c + cl;
                const f32x4 v = *reinterpret_cast<const f32x4 *>(sX + r * LD + cl);
                if (t0 + r < tok1 && d < P.D) {
                    TX *o = dx + (int64_t)(t0 + r) * P.dx.st + d;
                    if (vec_dx) {
                        typedef TX tx4 __attribute__((ext_vector_type(4)));
                        *reinterpret_cast<tx4 *>(o) = tx4{(TX)v[0], (TX)v[1], (TX)v[2], (TX)v[3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (d + e < P.D)
                                o[e] = (TX)v[e];
                    }
                }
            }
        }
    }
    if (P.gscale) {
        // workgroup sum of gu * u: d loss / d scale = -(1/scale) * (sum over all workgroups)
        __shared__ float red[SHM_W];
        for (int o = 32; o > 0; o >>= 1)
            gsu += __shfl_xor(gsu, o);
        if (lane == 0)
            red[w] = gsu;
        __syncthreads();
        if (threadIdx.x == 0) {
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < SHM_W; ++i)
                a += red[i];
            P.gscale[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = a;
        }
    }
}

// d loss / d scale = -(sum of the soft-hash backward's per-workgroup partials) / scale, summed in
// fp64 by one workgroup in a fixed order (deterministic, and no host round trip for the scale).
__global__ __launch_bounds__(256) void race_scale_grad(const float *part, int n, const float *scale, float *out)
{
    __shared__ double red[4];
    double a = 0.0;
    for (int i = threadIdx.x; i < n; i += 256)
        a += (double)part[i];
    for (int o = 32; o > 0; o >>= 1)
        a += __shfl_xor(a, o);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = a;
    __syncthreads();
    if (threadIdx.x == 0)
        out[0] = (float)(-(red[0] + red[1] + red[2] + red[3]) / (double)scale[0]);
}

hipError_t launch_scale_grad(const float *part, int n, const float *scale, float *out, hipStream_t s)
{
    hipLaunchKernelGGL(race_scale_grad, dim3(1), dim3(256), 0, s, part, n, scale, out);
    return hipGetLastError();
}

template <class TX, int KB, int NJT>
static const void *softhash_mfma_kernel(int bwd, int dp)
{
    if (bwd)
        return dp == 64 ? (const void *)race_softhash_bwd_mfma<TX, KB, NJT, 64>
                        : dp == 128 ? (const void *)race_softhash_bwd_mfma<TX, KB, NJT, 128>
                                    : (const void *)race_softhash_bwd_mfma<TX, KB, NJT, 256>;
    return dp == 64 ? (const void *)race_softhash_fwd_mfma<TX, KB, NJT, 64>
                    : dp == 128 ? (const void *)race_softhash_fwd_mfma<TX, KB, NJT, 128>
                                : (const void *)race_softhash_fwd_mfma<TX, KB, NJT, 256>;
}

// kernel of bit count K (1..4), plane tiles njt (1, 2) and head-dim class dp (64, 128, 256)
template <class TX>
static const void *softhash_mfma_kernel_k(int K, int bwd, int njt, int dp)
{
    switch (K * 2 + njt - 1) {
    case 2: return softhash_mfma_kernel<TX, 1, 1>(bwd, dp);
    case 3: return softhash_mfma_kernel<TX, 1, 2>(bwd, dp);
    case 4: return softhash_mfma_kernel<TX, 2, 1>(bwd, dp);
    case 5: return softhash_mfma_kernel<TX, 2, 2>(bwd, dp);
    case 6: return softhash_mfma_kernel<TX, 3, 1>(bwd, dp);
    case 7: return softhash_mfma_kernel<TX, 3, 2>(bwd, dp);
    case 8: return softhash_mfma_kernel<TX, 4, 1>(bwd, dp);
    case 9: return softhash_mfma_kernel<TX, 4, 2>(bwd, dp);
    default: return nullptr;
    }
}

// kernel of bit count K (1..8) for one direction, dtype and head-dim class (D <= 64, 128, 256)
template <class TX, int KB>
static const void *softhash_kernel(int bwd, int D)
{
    if (!bwd)
        return (const void *)race_softhash_fwd<TX, KB>;
    return D <= 64 ? (const void *)race_softhash_bwd<TX, KB, 2>
                   : D <= 128 ? (const void *)race_softhash_bwd<TX, KB, 4> : (const void *)race_softhash_bwd<TX, KB, 8>;
}

template <class TX>
static const void *softhash_kernel_k(int K, int bwd, int D)
{
    switch (K) {
    case 1: return softhash_kernel<TX, 1>(bwd, D);
    case 2: return softhash_kernel<TX, 2>(bwd, D);
    case 3: return softhash_kernel<TX, 3>(bwd, D);
    case 4: return softhash_kernel<TX, 4>(bwd, D);
    case 5: return softhash_kernel<TX, 5>(bwd, D);
    case 6: return softhash_kernel<TX, 6>(bwd, D);
    case 7: return softhash_kernel<TX, 7>(bwd, D);
    case 8: return softhash_kernel<TX, 8>(bwd, D);
    default: return nullptr;
    }
}

size_t softhash_smem(int D, int LK, bool bwd)
{
    const size_t DX = sh_dx(D);
    return sizeof(float) * (DX * sh_pl(LK) + SH_TT * DX + (size_t)SH_TT * LK + (bwd ? (size_t)SH_TT * sh_pg(LK) : 0));
}

// tokens per tile: SH_TT for the FMA kernels, one 16-token tile per wave for the matrix-core ones
static int softhash_tile(bool mf) { return mf ? SHM_W * 16 : SH_TT; }

int softhash_tiles_per_wg(int T, int B, int H, bool mf)
{
    // a workgroup walks up to 32 consecutive tiles of one (b, h) (planes loaded once), as long as
    // the grid keeps about 2048 workgroups (8 per CU; the FMA kernels) or 8192 (the matrix-core
    // kernels, about 5 resident per CU: several rounds, so the last one's tail is short)
    const int tile = softhash_tile(mf);
    const int64_t tiles = (int64_t)((T + tile - 1) / tile) * B * H;
    return (int)std::max<int64_t>(1, std::min<int64_t>(32, tiles / (mf ? 8192 : 2048)));
}

int softhash_grid_x(int T, int B, int H, bool mf)
{
    const int tile = softhash_tile(mf);
    const int ntt = (T + tile - 1) / tile, tpw = softhash_tiles_per_wg(T, B, H, mf);
    return (ntt + tpw - 1) / tpw;
}

hipError_t launch_softhash(const SoftHashParams &P, int bf16, int bwd, hipStream_t s)
{
    const bool mf = softhash_mfma_ok(P.D, P.L, P.K, P.M, bwd);
    const ShmLayout Y(P.D, P.LK);
    const void *fn = mf ? (bf16 ? softhash_mfma_kernel_k<__bf16>(P.K, bwd, Y.njt, Y.DX16)
                                : softhash_mfma_kernel_k<float>(P.K, bwd, Y.njt, Y.DX16))
                        : (bf16 ? softhash_kernel_k<__bf16>(P.K, bwd, P.D) : softhash_kernel_k<float>(P.K, bwd, P.D));
    if (!fn)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)softhash_grid_x(P.T, P.B, P.H, mf), (unsigned)(P.B * P.H),
                    (unsigned)(bwd ? 1 : (P.unshared ? P.M : 1)));
    const size_t smem = mf ? sizeof(float) * Y.floats(bwd) : softhash_smem(P.D, P.LK, bwd);
    SoftHashParams args = P;
    args.tpw = softhash_tiles_per_wg(P.T, P.B, P.H, mf);
    void *argv[] = {&args};
    return hipLaunchKernel(fn, grid, dim3(mf ? SHM_W * 64 : 256), argv, smem, s);
}

hipError_t softhash_prepare(int D, int LK)
{
    const int smem = (int)softhash_smem(D, LK, true);
    hipError_t e = hipSuccess;
    const ShmLayout Y(D, LK);
    const int smem_mf = (int)sizeof(float) * Y.floats(true);
    if (D <= 256 && LK <= 32 && smem_mf > 64 * 1024) {
        for (int K = 1; K <= 4 && e == hipSuccess; ++K)
            for (int bwd = 0; bwd < 2 && e == hipSuccess; ++bwd) {
                e = hipFuncSetAttribute(softhash_mfma_kernel_k<float>(K, bwd, Y.njt, Y.DX16),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, smem_mf);
                if (e == hipSuccess)
                    e = hipFuncSetAttribute(softhash_mfma_kernel_k<__bf16>(K, bwd, Y.njt, Y.DX16),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, smem_mf);
            }
    }
    if (smem > 64 * 1024) {
        for (int K = 1; K <= 8 && e == hipSuccess; ++K)
            for (int bwd = 0; bwd < 2 && e == hipSuccess; ++bwd) {
                e = hipFuncSetAttribute(softhash_kernel_k<float>(K, bwd, D), hipFuncAttributeMaxDynamicSharedMemorySize,
                                        smem);
                if (e == hipSuccess)
                    e = hipFuncSetAttribute(softhash_kernel_k<__bf16>(K, bwd, D),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, smem);
            }
    }
    return e;
}

// ============================================================================ decode
// One workgroup per (sequence b, kv head hk). State A [S], Bs [S][D] fp32 in HBM,
// updated in place: A += pK, Bs += pK (x) v (inclusive prefix: the new token is
// part of its own readout), then out_g = sum_s pQ_g[s] Bs[s,:] / (A[s] + eps)
// for the G query heads of the group.
template <class TX, int D, int GM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(GM <= 4 ? 8 : 1))) void race_decode_step(DecodeParams P)
{
    // thread layout of the state update: TPR threads per bucket row (VEC floats each), RIF
    // rows per pass over the state, PFR rows per thread loaded together; GM >= G query heads.
    // Registers stay within 64 per lane and LDS within 20 KB, so eight workgroups fit a CU
    // and a 256-CU device runs the 2048 (sequence, kv head) pairs of a decode batch in one round.
    constexpr int VEC = 4, TPR = D / VEC, RIF = 256 / TPR, PFR = 4, NWV = 4;
    extern __shared__ float sm[];
    const int G = P.G, LK = P.L * P.K, R = 1 << P.K, S = P.L * R;
    const bool pl_lds = D * LK <= DEC_PL_LDS;  // planes staged in LDS
    float *sIn = sm;                  // [G + 2][D]: k, v, q_0 .. q_{G-1}
    float *sU = sIn + (G + 2) * D;    // [G + 1][LK]: u for k, q_g
    float *sP = sU + (G + 1) * LK;    // [G + 1][S]: pK, pQ_g
    float *sRed = sP + (G + 1) * S;   // [NWV][G][D]: readout partial sums per wave
    float *sPl = sRed + NWV * G * D;  // [D][LK] planes (pl_lds)
    const int z = blockIdx.x;         // b * Hkv + hk
    const int b = z / P.Hkv, hk = z % P.Hkv;
    const int rr = threadIdx.x / TPR, dv = (threadIdx.x % TPR) * VEC;
    float *A = P.A + (int64_t)z * S;
    float *Bs = P.Bs + (int64_t)z * S * D;
    f32x4 bpre[PFR];
    float apre[PFR];
    // first PFR rows of this thread: loads of clamped rows (always inside the state), all in
    // flight together. Issued once no later global load has to be waited for before the update
    // (the memory counter is in order): after the planes are in LDS, or after the projections.
    auto prefetch_state = [&]() {
#pragma unroll
        for (int j = 0; j < PFR; ++j) {
            const int sr = min(rr + j * RIF, S - 1);
            bpre[j] = *reinterpret_cast<const f32x4 *>(Bs + (int64_t)sr * D + dv);
            apre[j] = A[sr];
        }
    };
    const TX *q = reinterpret_cast<const TX *>(P.q);
    const TX *k = reinterpret_cast<const TX *>(P.k);
    const TX *v = reinterpret_cast<const TX *>(P.v);
    for (int i = threadIdx.x; i < (G + 2) * D; i += 256) {
        const int row = i / D, d = i % D;
        float x;
        if (row == 0)
            x = (float)k[((int64_t)b * P.Hkv + hk) * D + d];
        else if (row == 1)
            x = (float)v[((int64_t)b * P.Hkv + hk) * D + d];
        else
            x = (float)q[((int64_t)b * P.Hkv * G + hk * G + (row - 2)) * D + d];
        sIn[row * D + d] = x;
    }
    if (pl_lds) {
        for (int i = threadIdx.x; i < D * LK; i += 256) {
            const float pl = P.planes[i];
            sPl[i] = P.round_planes ? (float)(__bf16)pl : pl;
        }
    }
    __syncthreads();
    if (pl_lds)
        prefetch_state();
    // projections: row 0 = k, rows 1.. = q_g
    for (int i = threadIdx.x; i < (G + 1) * LK; i += 256) {
        const int row = i / LK, j = i % LK;
        const float *x = sIn + (row == 0 ? 0 : row + 1) * D;
        float acc = 0.0f;
        if (pl_lds) {
            for (int d = 0; d < D; ++d)
                acc += x[d] * sPl[d * LK + j];
        } else {
#pragma unroll 8
            for (int d = 0; d < D; ++d) {
                const float pl = P.planes[d * LK + j];
                acc += x[d] * (P.round_planes ? (float)(__bf16)pl : pl);
            }
        }
        sU[row * LK + j] = tanh_f(acc) * P.inv_scale;
    }
    if (!pl_lds)
        prefetch_state();
    __syncthreads();
    for (int i = threadIdx.x; i < (G + 1) * P.L; i += 256) {
        const int row = i / P.L, l = i % P.L;
        float u[4], p[16];
        for (int kk = 0; kk < 4; ++kk)
            u[kk] = (kk < P.K) ? sU[row * LK + l * P.K + kk] : 0.0f;
        expand_probs(u, P.K, p);
        for (int r = 0; r < 16; ++r)
            if (r < R)
                sP[row * S + l * R + r] = p[r];
    }
    __syncthreads();
    // state update + readout, PFR rows per thread at a time
    float acc[GM][VEC];
    for (int g = 0; g < GM; ++g)
        for (int e = 0; e < VEC; ++e)
            acc[g][e] = 0.0f;
    float vv[VEC];
    for (int e = 0; e < VEC; ++e)
        vv[e] = sIn[D + dv + e];
    for (int s0 = 0; s0 < S; s0 += PFR * RIF) {
        if (s0 > 0) {
#pragma unroll
            for (int j = 0; j < PFR; ++j) {
                const int sr = min(s0 + rr + j * RIF, S - 1);
                bpre[j] = *reinterpret_cast<const f32x4 *>(Bs + (int64_t)sr * D + dv);
                apre[j] = A[sr];
            }
        }
#pragma unroll
        for (int j = 0; j < PFR; ++j) {
            const int s = s0 + rr + j * RIF;
            if (s < S) {
                const float pk = sP[s];
                const float a = apre[j] + pk;
                f32x4 bv = bpre[j];
                for (int e = 0; e < VEC; ++e)
                    bv[e] += pk * vv[e];
                *reinterpret_cast<f32x4 *>(Bs + (int64_t)s * D + dv) = bv;
                if (dv == 0)
                    A[s] = a;
                const float inv = frcp(a + P.eps);
                for (int g = 0; g < GM; ++g)
                    if (g < G) {
                        const float w = sP[(1 + g) * S + s] * inv;
                        for (int e = 0; e < VEC; ++e)
                            acc[g][e] += w * bv[e];
                    }
            }
        }
    }
    // the rows of one wave share the lanes' head-dim columns: lanes l, l + TPR, ... add up by
    // shuffles, then one partial sum per wave goes through LDS
    const int wv = threadIdx.x >> 6;
    for (int g = 0; g < GM; ++g)
        if (g < G)
            for (int e = 0; e < VEC; ++e) {
                float x = acc[g][e];
#pragma unroll
                for (int m = TPR; m < 64; m <<= 1)
                    x += __shfl_xor(x, m, 64);
                if ((threadIdx.x & 63) < TPR)
                    sRed[(wv * G + g) * D + dv + e] = x;
            }
    __syncthreads();
    TX *out = reinterpret_cast<TX *>(P.out);
    for (int i = threadIdx.x; i < G * D; i += 256) {
        const int g = i / D, d = i % D;
        float sum = 0.0f;
        for (int r = 0; r < NWV; ++r)
            sum += sRed[(r * G + g) * D + d];
        out[((int64_t)b * P.Hkv * G + hk * G + g) * D + d] = (TX)sum;
    }
}

// dynamic LDS of one decode workgroup (floats): inputs, soft bits, probabilities, partial sums
static size_t decode_smem(const DecodeParams &P)
{
    const int LK = P.L * P.K, S = P.L << P.K, NWV = 4;
    const size_t pl = P.D * LK <= DEC_PL_LDS ? (size_t)P.D * LK : 0;
    return sizeof(float) * ((size_t)(P.G + 2) * P.D + (size_t)(P.G + 1) * LK + (size_t)(P.G + 1) * S +
                            (size_t)NWV * P.G * P.D + pl);
}

hipError_t launch_decode(const DecodeParams &P, int bf16, hipStream_t s)
{
    const dim3 grid((unsigned)(P.B * P.Hkv));
    const size_t smem = decode_smem(P);
    if (smem > 64 * 1024)
        return hipErrorInvalidValue;
    if (P.G < 1 || P.G > DEC_GMAX)
        return hipErrorInvalidValue;
#define DEC(TX, DD, GM) hipLaunchKernelGGL((race_decode_step<TX, DD, GM>), grid, dim3(256), smem, s, P)
#define DEC_G(TX, DD)                 \
    if (P.G == 1) DEC(TX, DD, 1);     \
    else if (P.G == 2) DEC(TX, DD, 2); \
    else if (P.G <= 4) DEC(TX, DD, 4); \
    else DEC(TX, DD, 8)
    if (P.D == 64) {
        if (bf16) { DEC_G(__bf16, 64); } else { DEC_G(float, 64); }
    } else if (P.D == 128) {
        if (bf16) { DEC_G(__bf16, 128); } else { DEC_G(float, 128); }
    } else {
        return hipErrorInvalidValue;
    }
#undef DEC_G
#undef DEC
    return hipGetLastError();
}

// final state slot NB of a forward workspace -> dense decode state
__global__ void race_state_extract(const float *wsB, const float *wsA, int NB, int S_pad, int DPw,
                                   int S, int D, float *A, float *Bs, int64_t total)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total)
        return;
    const int d = (int)(i % (D + 1));
    const int64_t r = i / (D + 1);
    const int s = (int)(r % S);
    const int64_t z = r / S;
    const int64_t slot = z * (NB + 1) + NB;
    if (d == D)
        A[z * S + s] = wsA[slot * S_pad + s];
    else
        Bs[(z * S + s) * D + d] = wsB[(slot * S_pad + s) * DPw + d];
}

hipError_t launch_state_extract(const float *wsB, const float *wsA, int NB, int S_pad, int DPw,
                                int Z, int S, int D, float *A, float *Bs, hipStream_t s)
{
    const int64_t total = (int64_t)Z * S * (D + 1);
    hipLaunchKernelGGL(race_state_extract, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       wsB, wsA, NB, S_pad, DPw, S, D, A, Bs, total);
    return hipGetLastError();
}

}  // namespace race
