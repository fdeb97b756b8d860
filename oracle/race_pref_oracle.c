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
 *  orc_race_windows         the same forward/backward for one long stream with
 *                           the buckets split over threads, an optional carried-in
 *                           prefix state, and outputs kept only on token windows.
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

/*
 * orc_race_windows: one stream of the same streaming fp64 forward/backward as
 * orc_race_fwd / orc_race_bwd (race_common.py:76-90; backward_kernels.cu:10-17),
 * for long sequences where only some token windows are compared. The buckets are
 * split over the OpenMP threads (every bucket's scan is independent; the outputs
 * that sum over buckets are reduced at the end), so one stream of 2^20 tokens at
 * S = 128 runs in seconds.
 *   pK, pQ [T][S], V [T][D], gO [T][D] or NULL (forward only);
 *   A0 [S], B0 [S][D] or NULL: bucket state carried in before token 0 (the
 *     sequence's earlier tokens), so a late window of a long sequence is checked
 *     from its exact prefix state;
 *   wins [nwin] sorted, non-overlapping window starts, each [w, w + wlen) in [0, T);
 *   out_w [nwin][wlen][D]; with gO also gpK_w, gpQ_w [nwin][wlen][S], gV_w [nwin][wlen][D]
 *   (the suffix sums of the backward run over [0, T)).
 */
#include <omp.h>

void orc_race_windows(const double *pK, const double *pQ, const double *V, const double *gO,
                      int64_t T, int64_t S, int64_t D, double eps, const double *A0,
                      const double *B0, const int64_t *wins, int64_t nwin, int64_t wlen,
                      double *out_w, double *gpK_w, double *gpQ_w, double *gV_w)
{
    int32_t *widx = (int32_t *)malloc((size_t)T * sizeof(int32_t));
    for (int64_t t = 0; t < T; ++t)
        widx[t] = -1;
    for (int64_t w = 0; w < nwin; ++w)
        for (int64_t i = 0; i < wlen; ++i)
            widx[wins[w] + i] = (int32_t)(w * wlen + i);
    const int64_t nrow = nwin * wlen;
    int nth = omp_get_max_threads();
    if (nth > S)
        nth = (int)S;
    double *part_out = (double *)calloc((size_t)(nth * nrow * D), sizeof(double));
    double *part_gv = gO ? (double *)calloc((size_t)(nth * nrow * D), sizeof(double)) : NULL;
#pragma omp parallel num_threads(nth)
    {
        const int id = omp_get_thread_num();
        const int64_t s0 = S * id / nth, s1 = S * (id + 1) / nth, ns = s1 - s0;
        double *A = (double *)calloc((size_t)ns, sizeof(double));
        double *B = (double *)calloc((size_t)(ns * D), sizeof(double));
        double *W = gO ? (double *)malloc((size_t)(T * ns) * sizeof(double)) : NULL;
        double *gA = gO ? (double *)malloc((size_t)(T * ns) * sizeof(double)) : NULL;
        double *po = part_out + id * nrow * D;
        if (A0)
            for (int64_t j = 0; j < ns; ++j)
                A[j] = A0[s0 + j];
        if (B0)
            memcpy(B, B0 + s0 * D, (size_t)(ns * D) * sizeof(double));
        for (int64_t t = 0; t < T; ++t) {
            const int32_t wi = widx[t];
            const double *v = V + t * D;
            const double *go = gO ? gO + t * D : NULL;
            for (int64_t j = 0; j < ns; ++j) {
                const int64_t s = s0 + j;
                const double pk = pK[t * S + s];
                A[j] += pk;
                double *b = B + j * D;
                double gw = 0.0;
                if (go) {
                    for (int64_t d = 0; d < D; ++d) {
                        b[d] += pk * v[d];
                        gw += go[d] * b[d];
                    }
                } else {
                    for (int64_t d = 0; d < D; ++d)
                        b[d] += pk * v[d];
                }
                const double inv = 1.0 / (A[j] + eps);
                const double w = pQ[t * S + s] * inv;
                if (go) {
                    W[t * ns + j] = w;
                    gA[t * ns + j] = -w * gw * inv;
                }
                if (wi >= 0) {
                    double *o = po + (int64_t)wi * D;
                    for (int64_t d = 0; d < D; ++d)
                        o[d] += w * b[d];
                    if (go)
                        gpQ_w[(int64_t)wi * S + s] = gw * inv;
                }
            }
        }
        if (gO) {
            double *pg = part_gv + id * nrow * D;
            memset(A, 0, (size_t)ns * sizeof(double));
            memset(B, 0, (size_t)(ns * D) * sizeof(double));
            for (int64_t t = T - 1; t >= 0; --t) {
                const int32_t wi = widx[t];
                const double *v = V + t * D;
                const double *go = gO + t * D;
                for (int64_t j = 0; j < ns; ++j) {
                    A[j] += gA[t * ns + j];
                    double *gb = B + j * D;
                    const double w = W[t * ns + j];
                    for (int64_t d = 0; d < D; ++d)
                        gb[d] += w * go[d];
                    if (wi >= 0) {
                        const double pk = pK[t * S + s0 + j];
                        double dot = 0.0, *g = pg + (int64_t)wi * D;
                        for (int64_t d = 0; d < D; ++d) {
                            dot += gb[d] * v[d];
                            g[d] += pk * gb[d];
                        }
                        gpK_w[(int64_t)wi * S + s0 + j] = A[j] + dot;
                    }
                }
            }
        }
        free(A);
        free(B);
        free(W);
        free(gA);
    }
    for (int64_t i = 0; i < nrow * D; ++i) {
        double so = 0.0, sg = 0.0;
        for (int k = 0; k < nth; ++k) {
            so += part_out[k * nrow * D + i];
            if (gO)
                sg += part_gv[k * nrow * D + i];
        }
        out_w[i] = so;
        if (gO)
            gV_w[i] = sg;
    }
    free(part_out);
    free(part_gv);
    free(widx);
}
