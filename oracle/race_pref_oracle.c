/*
 * C restatement of the reference's CPU RACE kernels -- TEST INFRASTRUCTURE ONLY.
 *
 * Built into oracle/liborace.so by oracle/Makefile and loaded with ctypes by
 * oracle/oracle_c.py. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it; the HIP product never links or calls it.
 *
 *  orc_prefix_mean_flat     restates kernels/cpu/race_pref.cpp:36-101
 *                           (per stream: A += w; B += w*v; E = B/(A+eps);
 *                            fp64 accumulation, fp32 store)
 *  orc_prefix_mean_flat_bw  restates kernels/cpu/race_pref.cpp:104-220
 *                           (forward pass for invA/alpha, reverse pass with the
 *                            suffix sums beta_suf / alpha_suf)
 *  orc_race_fwd             streaming fp64 form of race_common.py:76-90 over the
 *                           collapsed buckets S: O(S*D) state per stream, so long
 *                           T can be checked without the [N,T,S,D] cumsum.
 *  orc_race_bwd             streaming fp64 form of the exact backward written in
 *                           kernels/gpu/backward_kernels.cu:10-17:
 *                             gW = <go, B_t>; gpQ = gW/(A+eps);
 *                             gA = -pQ*gW/(A+eps)^2; gB = pQ*go/(A+eps);
 *                             suffix sums gAn, gBn; gpK = gAn + <gBn, v>;
 *                             gv = sum_s pK * gBn.
 * Pinned in tests/test_oracle.py against torch fp64 autograd, gradcheck and the
 * compiled reference kernel (oracle/_ref) when that is built.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

void orc_prefix_mean_flat(const float *pk, const float *v, float *E,
                          int64_t NS, int64_t T, int64_t D, double eps)
{
#pragma omp parallel for schedule(static)
    for (int64_t ns = 0; ns < NS; ++ns) {
        double A = 0.0;
        double *B = (double *)calloc((size_t)D, sizeof(double));
        const float *w = pk + ns * T;
        const float *vs = v + ns * T * D;
        float *es = E + ns * T * D;
        for (int64_t t = 0; t < T; ++t) {
            const float wt = w[t];
            A += (double)wt;
            const double inv = 1.0 / (A + eps);
            for (int64_t d = 0; d < D; ++d) {
                B[d] += (double)wt * (double)vs[t * D + d];
                es[t * D + d] = (float)(B[d] * inv);
            }
        }
        free(B);
    }
}

void orc_prefix_mean_flat_bw(const float *w, const float *v, const float *gE,
                             float *gW, float *gV, int64_t NS, int64_t T, int64_t D,
                             double eps)
{
#pragma omp parallel for schedule(static)
    for (int64_t ns = 0; ns < NS; ++ns) {
        const float *ws = w + ns * T;
        const float *vs = v + ns * T * D;
        const float *gs = gE + ns * T * D;
        float *gws = gW + ns * T;
        float *gvs = gV + ns * T * D;
        double *invA = (double *)malloc((size_t)T * sizeof(double));
        double *alpha = (double *)malloc((size_t)T * sizeof(double));
        double *B = (double *)calloc((size_t)D, sizeof(double));
        double *beta = (double *)calloc((size_t)D, sizeof(double));
        double A = 0.0;
        for (int64_t t = 0; t < T; ++t) {
            const double wt = (double)ws[t];
            A += wt;
            for (int64_t d = 0; d < D; ++d)
                B[d] += wt * (double)vs[t * D + d];
            const double iA = 1.0 / (A + eps);
            invA[t] = iA;
            double dot = 0.0;
            for (int64_t d = 0; d < D; ++d)
                dot += (double)gs[t * D + d] * B[d];
            alpha[t] = -(iA * iA) * dot;
        }
        double alpha_suf = 0.0;
        for (int64_t t = T - 1; t >= 0; --t) {
            const double iA = invA[t];
            for (int64_t d = 0; d < D; ++d)
                beta[d] += (double)gs[t * D + d] * iA;
            alpha_suf += alpha[t];
            double dot = 0.0;
            for (int64_t d = 0; d < D; ++d)
                dot += beta[d] * (double)vs[t * D + d];
            gws[t] = (float)(alpha_suf + dot);
            const double wt = (double)ws[t];
            for (int64_t d = 0; d < D; ++d)
                gvs[t * D + d] = (float)(wt * beta[d]);
        }
        free(invA);
        free(alpha);
        free(B);
        free(beta);
    }
}

void orc_race_fwd(const double *pK, const double *pQ, const double *V, double *out,
                  double *Afin, double *Bfin, int64_t N, int64_t T, int64_t S, int64_t D,
                  double eps)
{
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t n = 0; n < N; ++n) {
        double *A = (double *)calloc((size_t)S, sizeof(double));
        double *B = (double *)calloc((size_t)(S * D), sizeof(double));
        for (int64_t t = 0; t < T; ++t) {
            const double *pk = pK + (n * T + t) * S;
            const double *pq = pQ + (n * T + t) * S;
            const double *v = V + (n * T + t) * D;
            double *o = out + (n * T + t) * D;
            for (int64_t d = 0; d < D; ++d)
                o[d] = 0.0;
            for (int64_t s = 0; s < S; ++s) {
                A[s] += pk[s];
                const double w = pq[s] / (A[s] + eps);
                double *b = B + s * D;
                for (int64_t d = 0; d < D; ++d) {
                    b[d] += pk[s] * v[d];
                    o[d] += w * b[d];
                }
            }
        }
        if (Afin)
            memcpy(Afin + n * S, A, (size_t)S * sizeof(double));
        if (Bfin)
            memcpy(Bfin + n * S * D, B, (size_t)(S * D) * sizeof(double));
        free(A);
        free(B);
    }
}

void orc_race_bwd(const double *pK, const double *pQ, const double *V, const double *gO,
                  double *gpK, double *gpQ, double *gV, int64_t N, int64_t T, int64_t S,
                  int64_t D, double eps)
{
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t n = 0; n < N; ++n) {
        double *A = (double *)calloc((size_t)S, sizeof(double));
        double *B = (double *)calloc((size_t)(S * D), sizeof(double));
        double *gA = (double *)malloc((size_t)(T * S) * sizeof(double));
        double *W = (double *)malloc((size_t)(T * S) * sizeof(double));
        /* forward pass: rebuild A_t, B_t; gW, gpQ, gA, W per token */
        for (int64_t t = 0; t < T; ++t) {
            const double *pk = pK + (n * T + t) * S;
            const double *pq = pQ + (n * T + t) * S;
            const double *v = V + (n * T + t) * D;
            const double *go = gO + (n * T + t) * D;
            for (int64_t s = 0; s < S; ++s) {
                A[s] += pk[s];
                double *b = B + s * D;
                double gw = 0.0;
                for (int64_t d = 0; d < D; ++d) {
                    b[d] += pk[s] * v[d];
                    gw += go[d] * b[d];
                }
                const double inv = 1.0 / (A[s] + eps);
                gpQ[(n * T + t) * S + s] = gw * inv;
                gA[t * S + s] = -pq[s] * gw * inv * inv;
                W[t * S + s] = pq[s] * inv;
            }
        }
        /* reverse pass: suffix sums gAn[S], gBn[S,D] */
        double *gAn = A;
        double *gBn = B;
        memset(gAn, 0, (size_t)S * sizeof(double));
        memset(gBn, 0, (size_t)(S * D) * sizeof(double));
        for (int64_t t = T - 1; t >= 0; --t) {
            const double *pk = pK + (n * T + t) * S;
            const double *v = V + (n * T + t) * D;
            const double *go = gO + (n * T + t) * D;
            double *gv = gV + (n * T + t) * D;
            for (int64_t d = 0; d < D; ++d)
                gv[d] = 0.0;
            for (int64_t s = 0; s < S; ++s) {
                gAn[s] += gA[t * S + s];
                double *gb = gBn + s * D;
                const double w = W[t * S + s];
                double dot = 0.0;
                for (int64_t d = 0; d < D; ++d) {
                    gb[d] += w * go[d];
                    dot += gb[d] * v[d];
                    gv[d] += pk[s] * gb[d];
                }
                gpK[(n * T + t) * S + s] = gAn[s] + dot;
            }
        }
        free(A);
        free(B);
        free(gA);
        free(W);
    }
}
