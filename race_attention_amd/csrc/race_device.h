// Device building blocks for the causal RACE kernels on CDNA4 (gfx950).
//
//  * Two MFMA "engines" share one tile interface:
//      EngBF16  v_mfma_f32_16x16x32_bf16  (bf16 operands in LDS, fp32 accumulate)
//      EngF32   v_mfma_f32_16x16x4_f32    (fp32 operands in LDS, fp32 accumulate)
//    A 16x16 output tile is owned by one wave64. Lane l holds rows
//    (l>>4)*4 + e (e = 0..3) of column (l&15). Operand fragments are read from LDS
//    buffers stored "k-contiguous": A as [m][k], B as [n][k] (lane l reads row
//    l&15 at k offset (l>>4)*KPL).
//  * Soft-hash math of scaling/race_common.py:56-72 in closed form:
//      u_k = tanh(x . plane_k) / scale,
//      p[r] = prod_k sigmoid(2 c_k(r) u_k),  c_k(r) = +1 iff bit (K-1-k) of r,
//    which equals the reference's softmax over the 2^K corner logits
//    sum_k c_k(r) u_k (the partition function factorises over the bits).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define RACE_DEV __device__ __forceinline__

namespace race {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------ engines
struct EngBF16 {
    typedef __bf16 T;
    typedef bf16x8 frag;
    static constexpr int KSTEP = 32;  // k per MFMA
    static constexpr int KPL = 8;     // k elements per lane
    static constexpr int PAD = 8;     // LDS row padding (elements): 16 bytes
    static RACE_DEV frag ld(const T *p) { return *reinterpret_cast<const frag *>(p); }
    static RACE_DEV void mma(f32x4 &c, const frag &a, const frag &b)
    {
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    static RACE_DEV frag neg(frag a)
    {
        u32x4 u = __builtin_bit_cast(u32x4, a);
        u ^= 0x80008000u;
        return __builtin_bit_cast(frag, u);
    }
    static RACE_DEV T cvt(float x) { return (T)x; }
    // fragment of a 0/1 (or 0/val) matrix M[m][k] generated in registers
    template <class Pred>
    static RACE_DEV frag gen(int m, int kbase, Pred pred, float val)
    {
        frag f;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            f[e] = (T)(pred(m, kbase + e) ? val : 0.0f);
        return f;
    }
};

struct EngF32 {
    typedef float T;
    typedef float frag;
    static constexpr int KSTEP = 4;
    static constexpr int KPL = 1;
    static constexpr int PAD = 4;
    static RACE_DEV frag ld(const T *p) { return *p; }
    static RACE_DEV void mma(f32x4 &c, const frag &a, const frag &b)
    {
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
    static RACE_DEV frag neg(frag a) { return -a; }
    static RACE_DEV T cvt(float x) { return x; }
    template <class Pred>
    static RACE_DEV frag gen(int m, int kbase, Pred pred, float val)
    {
        return pred(m, kbase) ? val : 0.0f;
    }
};

// acc += A[m0..m0+16, 0..K) * B[n0..n0+16, 0..K)^T   (A: [m][k] lda, B: [n][k] ldb)
template <class E, int K, bool NEG_A = false>
RACE_DEV void mma_tile(f32x4 &acc, const typename E::T *A, int lda, const typename E::T *B,
                       int ldb, int m0, int n0, int lane)
{
    const typename E::T *pa = A + (m0 + (lane & 15)) * lda + (lane >> 4) * E::KPL;
    const typename E::T *pb = B + (n0 + (lane & 15)) * ldb + (lane >> 4) * E::KPL;
#pragma unroll
    for (int k = 0; k < K; k += E::KSTEP) {
        typename E::frag a = E::ld(pa + k);
        if (NEG_A)
            a = E::neg(a);
        E::mma(acc, a, E::ld(pb + k));
    }
}

// acc += G[m0.., 0..K) * B[n0.., 0..K)^T where G is generated in registers by pred
template <class E, int K, class Pred>
RACE_DEV void mma_tile_gen(f32x4 &acc, Pred pred, float val, const typename E::T *B, int ldb,
                           int m0, int n0, int lane)
{
    const typename E::T *pb = B + (n0 + (lane & 15)) * ldb + (lane >> 4) * E::KPL;
    const int m = m0 + (lane & 15);
#pragma unroll
    for (int k = 0; k < K; k += E::KSTEP)
        E::mma(acc, E::template gen<Pred>(m, k + (lane >> 4) * E::KPL, pred, val), E::ld(pb + k));
}

// accumulator coordinates
RACE_DEV int acc_row(int m0, int lane) { return m0 + ((lane >> 4) << 2); }
RACE_DEV int acc_col(int n0, int lane) { return n0 + (lane & 15); }

// store an accumulator tile into LDS, row-major [row][col]
template <class T>
RACE_DEV void st_rm(T *buf, int ld, int m0, int n0, int lane, const f32x4 &v)
{
    const int r = acc_row(m0, lane), c = acc_col(n0, lane);
#pragma unroll
    for (int e = 0; e < 4; ++e)
        buf[(r + e) * ld + c] = (T)v[e];
}
// store an accumulator tile into LDS, column-major [col][row] (one vector store)
RACE_DEV void st_cm(__bf16 *buf, int ld, int m0, int n0, int lane, const f32x4 &v)
{
    const int r = acc_row(m0, lane), c = acc_col(n0, lane);
    bf16x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        w[e] = (__bf16)v[e];
    *reinterpret_cast<bf16x4 *>(buf + c * ld + r) = w;
}
RACE_DEV void st_cm(float *buf, int ld, int m0, int n0, int lane, const f32x4 &v)
{
    const int r = acc_row(m0, lane), c = acc_col(n0, lane);
    *reinterpret_cast<f32x4 *>(buf + c * ld + r) = v;
}

// ------------------------------------------------------------------ scalar math
RACE_DEV float frcp(float x) { return __builtin_amdgcn_rcpf(x); }

// tanh(x) = 1 - 2 / (exp(2x) + 1); saturates to +-1 through exp overflow/underflow
RACE_DEV float tanh_f(float x) { return 1.0f - 2.0f * frcp(__expf(2.0f * x) + 1.0f); }

// Argument of a corner sigmoid, clamped to |u| <= lim: u = tanh(proj) / scale grows without
// bound as scale -> 0, and exp(-2u) must stay finite so that 1 / (1 + e) and e / (1 + e) never
// meet inf * 0. With lim = 40 the clamp moves a probability by at most e^-80 (the per-bit
// sigmoids below); the fused kernels' one-denominator form needs (1 + e^(2 lim))^4 finite and
// uses lim = 10 (a shift of at most 2e-9, below fp32 resolution next to 1).
RACE_DEV float sig_arg(float u, float lim = 40.0f) { return __builtin_amdgcn_fmed3f(u, -lim, lim); }

// Probabilities of one hash table from its K soft bits u[0..K):
// p[r] = prod_k sigmoid(2 c_k(r) u_k), r < 2^K (K <= 4).  Bit k = 0 is the most
// significant bit of r, matching itertools.product([-1, 1], repeat=K).
RACE_DEV void expand_probs(const float *u, int K, float p[16])
{
    p[0] = 1.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (k < K) {
            const float e = __expf(-2.0f * sig_arg(u[k]));
            const float s1 = frcp(1.0f + e);  // sigmoid(+2u): corner bit set
            const float s0 = e * s1;          // sigmoid(-2u): corner bit clear
            const int n = 1 << k;
#pragma unroll
            for (int i = n - 1; i >= 0; --i) {
                const float pi = p[i];
                p[2 * i + 1] = pi * s1;
                p[2 * i] = pi * s0;
            }
        }
    }
}

// Backward of one table: given u[K], p[R] and dL/dp[R], returns dL/dproj[K]
// through the softmax (dz = p (gp - <p,gp>)), the corner matrix (du_k =
// sum_r dz_r c_k(r)) and u = tanh(proj)/scale (dproj = du/scale (1 - tanh^2)).
RACE_DEV void softhash_bwd(const float *u, const float *p, const float *gp, int K, float scale,
                           float inv_scale, float *gproj)
{
    const int R = 1 << K;
    float dot = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r)
        if (r < R)
            dot += p[r] * gp[r];
    float gu[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        if (r < R) {
            const float gz = p[r] * (gp[r] - dot);
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (k < K)
                    gu[k] += ((r >> (K - 1 - k)) & 1) ? gz : -gz;
        }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (k < K) {
            const float th = u[k] * scale;
            gproj[k] = gu[k] * inv_scale * (1.0f - th * th);
        }
}

// ------------------------------------------------------------------ global I/O
RACE_DEV float ld_elem(const float *p) { return *p; }
RACE_DEV float ld_elem(const __bf16 *p) { return (float)*p; }
RACE_DEV void st_elem(float *p, float v) { *p = v; }
RACE_DEV void st_elem(__bf16 *p, float v) { *p = (__bf16)v; }

}  // namespace race
