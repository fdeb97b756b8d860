/*
 * race_attention.h -- C ABI of the MI355X (gfx950) causal RACE attention library
 * (librace_amd.so). Plain pointers, sizes and a stream handle; no C++ or torch
 * types cross this boundary. Every call is asynchronous on `stream` (a
 * hipStream_t; NULL is the null stream), allocates nothing, and returns a
 * race_status; race_last_error() gives the message of the last failure on the
 * calling thread.
 *
 * Reference interfaces replaced (sahiljoshi515/RACE_Attention):
 *   race_soft_hash_fwd/bwd  scaling/race_common.py:36-73  soft_hash_probs (+ its autograd)
 *   race_op_fwd             kernels/gpu/forward_kernel.cu:110-137  race_fused_fwd
 *                           (bound at kernels/gpu/race_cuda_binding.cpp:12,18)
 *   race_op_bwd             kernels/gpu/backward_kernels.cu:174-215  race_backward
 *                           (bound at kernels/gpu/race_cuda_binding.cpp:13-14,21)
 *   race_qkv_fwd/bwd        scaling/race_causal_cuda.py:94-102 RaceCausalCuda.forward
 *                           (soft-hash + RaceCausalFn, race_causal_cuda.py:47-69) and its
 *                           backward, fused: q,k,v in, out / dq,dk,dv out
 *   race_qkv_final_state    the (A_final, B_final) returned by race_prefix_ref,
 *                           scaling/race_common.py:88-90
 *   race_decode_step        no reference counterpart (chat/nanochat/gpt.py:143-146 raises);
 *                           single-token step on the carried (A, B) state
 */
#ifndef RACE_ATTENTION_H
#define RACE_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RACE_ABI_VERSION 2  /* 2: kept-state entry points take the state's size */

typedef enum {
    RACE_OK = 0,
    RACE_ERR_INVALID = 1,     /* bad shape, pointer, stride or argument */
    RACE_ERR_UNSUPPORTED = 2, /* valid but not compiled for (e.g. head dim) */
    RACE_ERR_WORKSPACE = 3,   /* workspace missing or too small */
    RACE_ERR_HIP = 4          /* HIP runtime error while launching */
} race_status;

typedef enum { RACE_F32 = 0, RACE_BF16 = 1 } race_dtype;

typedef void *race_stream; /* hipStream_t */

/* A [B][H][T][D] tensor with contiguous last dimension; strides in elements. */
typedef struct {
    void *data;
    int64_t stride_b, stride_h, stride_t;
} race_tensor;

int race_abi_version(void);
const char *race_last_error(void);

/* ---------------------------------------------------------------- soft-hash */
typedef struct {
    int B, H, T, D; /* x is [B][H][T][D] */
    int L, K;       /* L tables of K bits: S = L * 2^K buckets */
    int M;          /* ensemble copies (N = M*B*H rows of probabilities) */
    int unshared;   /* 1: planes_T is [M][D][L*K] (share_planes=False), else [D][L*K] */
    float scale;    /* logits divisor; the reference uses sqrt(D) */
} race_hash_shape;

/* probs [Mp][B*H][T][L*2^K] fp32, Mp = M if unshared else 1 (shared planes give
 * identical rows for every ensemble copy). x fp32 or bf16; bf16 rounds the planes
 * to bf16 as the reference does (race_common.py:54). */
int race_soft_hash_fwd(const race_hash_shape *sh, race_tensor x, int x_dtype,
                       const float *planes_T, float *probs, race_stream stream);
/* dx (dtype of x, layout of dx) from gprobs [M][B*H][T][L*2^K] (summed over M). */
int race_soft_hash_bwd(const race_hash_shape *sh, race_tensor x, int x_dtype,
                       const float *planes_T, const float *gprobs, race_tensor dx,
                       race_stream stream);

/* As race_soft_hash_bwd, and also the temperature gradient of a learnable scale
 * (scaling/benchmark_time.py:104,111, logits = tanh(proj) / scale): gscale_partials
 * receives race_soft_hash_bwd_partials(sh) per-workgroup sums of (dL/du) * u with
 * u = tanh(proj) / scale, so dL/dscale = -(sum of the partials) / scale. */
int race_soft_hash_bwd_partials(const race_hash_shape *sh);
int race_soft_hash_bwd_scale(const race_hash_shape *sh, race_tensor x, int x_dtype,
                             const float *planes_T, const float *gprobs, race_tensor dx,
                             float *gscale_partials, race_stream stream);

/* race_soft_hash_fwd / race_soft_hash_bwd_scale with the scale read on the device from
 * scale_dev (one fp32 > 0; sh->scale is ignored), for the learnable temperature of the
 * non-causal BatchedACE (scaling/benchmark_time.py:104,111: scale =
 * exp(logit_temp).clamp(1e-2, 10), a device tensor that the reference's torch autograd never
 * reads back to the host). The backward also reduces its partials on the device:
 * dscale[0] = -(sum of the race_soft_hash_bwd_partials(sh) partials) / scale_dev[0], summed in
 * fp64 in a fixed order. Neither call synchronises, so both can be captured in a HIP graph. */
int race_soft_hash_fwd_dscale(const race_hash_shape *sh, race_tensor x, int x_dtype,
                              const float *planes_T, const float *scale_dev, float *probs,
                              race_stream stream);
int race_soft_hash_bwd_dscale(const race_hash_shape *sh, race_tensor x, int x_dtype,
                              const float *planes_T, const float *scale_dev,
                              const float *gprobs, race_tensor dx, float *gscale_partials,
                              float *dscale, race_stream stream);

/* ---------------------------------------------------------------- op-level scan */
/* pK, pQ [N][T][S], V / out / gO / gV [N][T][D], gpK / gpQ [N][T][S]; fp32,
 * contiguous. `block` = tokens per workgroup (0: automatic; results do not depend
 * on it beyond fp32 rounding). */
size_t race_op_workspace_bytes(int64_t N, int64_t T, int64_t S, int64_t D, int64_t block,
                               int backward);
int race_op_fwd(const float *pK, const float *pQ, const float *V, float *out, int64_t N,
                int64_t T, int64_t S, int64_t D, float eps, int64_t block, void *workspace,
                size_t workspace_bytes, race_stream stream);
int race_op_bwd(const float *pK, const float *pQ, const float *V, const float *gO, float *gpK,
                float *gpQ, float *gV, int64_t N, int64_t T, int64_t S, int64_t D, float eps,
                int64_t block, void *workspace, size_t workspace_bytes, race_stream stream);
/* race_op_fwd that also leaves its scanned forward block states in `state`
 * (race_op_state_bytes bytes, 256-byte aligned), and race_op_bwd that reads them from there
 * instead of recomputing them (same pK, V, shape and block as the forward; the backward only
 * reads the state, so it serves any number of backward calls). `state_bytes` is the buffer's
 * size; both calls fail with RACE_ERR_WORKSPACE when it is below race_op_state_bytes of their
 * own (N, T, S, D, block), so a buffer sized for another shape or block is never overrun.
 * No counterpart in the reference, whose backward (kernels/gpu/backward_kernels.cu:174-215)
 * recomputes the forward block states: for autograd callers that keep the forward's state
 * until the backward. */
size_t race_op_state_bytes(int64_t N, int64_t T, int64_t S, int64_t D, int64_t block);
int race_op_fwd_keep(const float *pK, const float *pQ, const float *V, float *out, int64_t N,
                     int64_t T, int64_t S, int64_t D, float eps, int64_t block, void *workspace,
                     size_t workspace_bytes, float *state, size_t state_bytes, race_stream stream);
int race_op_bwd_kept(const float *pK, const float *pQ, const float *V, const float *gO, float *gpK,
                     float *gpQ, float *gV, int64_t N, int64_t T, int64_t S, int64_t D, float eps,
                     int64_t block, void *workspace, size_t workspace_bytes, const float *state,
                     size_t state_bytes, race_stream stream);

/* ---------------------------------------------------------------- causal linear attention */
/* Katharopoulos causal linear attention, the reference's comparison kernel
 * (kernels/cpu/linear_pref.cpp:87-213, causal_dot_product / causal_dot_backward):
 * out_l = Q_l . sum_{s<=l} K_s (x) V_s, with Q, K [N][L][E], V / out / gO / gV [N][L][M]
 * and gQ, gK [N][L][E] fp32 contiguous (N = batch * heads). Runs on the causal scan
 * kernels with the normalisation removed; workspace from race_op_workspace_bytes(N, L,
 * E, M, block, backward). */
int race_causal_dot_product(const float *Q, const float *K, const float *V, float *out,
                            int64_t N, int64_t L, int64_t E, int64_t M, int64_t block,
                            void *workspace, size_t workspace_bytes, race_stream stream);
int race_causal_dot_backward(const float *Q, const float *K, const float *V, const float *gO,
                             float *gQ, float *gK, float *gV, int64_t N, int64_t L, int64_t E,
                             int64_t M, int64_t block, void *workspace, size_t workspace_bytes,
                             race_stream stream);
/* The same pair keeping the forward's block states in `state` (race_op_state_bytes(N, L, E, M,
 * block) bytes, 256-byte aligned, its size in `state_bytes`, checked as for race_op_fwd_keep)
 * for a backward that reads them instead of recomputing them; bitwise the same results. No
 * counterpart in the reference (linear_pref.cpp:138-213 recomputes the running sums in its
 * backward): for autograd callers that keep the state. */
int race_causal_dot_product_keep(const float *Q, const float *K, const float *V, float *out,
                                 int64_t N, int64_t L, int64_t E, int64_t M, int64_t block,
                                 void *workspace, size_t workspace_bytes, float *state,
                                 size_t state_bytes, race_stream stream);
int race_causal_dot_backward_kept(const float *Q, const float *K, const float *V, const float *gO,
                                  float *gQ, float *gK, float *gV, int64_t N, int64_t L, int64_t E,
                                  int64_t M, int64_t block, void *workspace,
                                  size_t workspace_bytes, const float *state, size_t state_bytes,
                                  race_stream stream);

/* ---------------------------------------------------------------- non-causal op */
/* Non-causal RACE of BatchedACE (scaling/benchmark_time.py:139-160), replacing its
 * torch bmm sequence: E = (pK^T V) / (sum_t pK + eps), out = pQ E; the backward
 * gives gpK, gpQ, gV as the autograd of that sequence. Same layouts and workspace
 * convention as race_op_*. */
size_t race_nc_op_workspace_bytes(int64_t N, int64_t T, int64_t S, int64_t D, int64_t block,
                                  int backward);
int race_nc_op_fwd(const float *pK, const float *pQ, const float *V, float *out, int64_t N,
                   int64_t T, int64_t S, int64_t D, float eps, int64_t block, void *workspace,
                   size_t workspace_bytes, race_stream stream);
int race_nc_op_bwd(const float *pK, const float *pQ, const float *V, const float *gO,
                   float *gpK, float *gpQ, float *gV, int64_t N, int64_t T, int64_t S,
                   int64_t D, float eps, int64_t block, void *workspace,
                   size_t workspace_bytes, race_stream stream);
/* The same pair keeping the forward's whole-sequence totals (sum pK, sum pK v) in `state`
 * (race_op_state_bytes bytes, 256-byte aligned, its size in `state_bytes`, checked as for
 * race_op_fwd_keep) for a backward that reads them instead of recomputing them; bitwise the
 * same results. No counterpart in the reference, whose BatchedACE backward (torch autograd,
 * scaling/benchmark_time.py:139-160) keeps the totals as saved tensors: for autograd callers
 * that keep the state until the backward. */
int race_nc_op_fwd_keep(const float *pK, const float *pQ, const float *V, float *out, int64_t N,
                        int64_t T, int64_t S, int64_t D, float eps, int64_t block, void *workspace,
                        size_t workspace_bytes, float *state, size_t state_bytes, race_stream stream);
int race_nc_op_bwd_kept(const float *pK, const float *pQ, const float *V, const float *gO,
                        float *gpK, float *gpQ, float *gV, int64_t N, int64_t T, int64_t S,
                        int64_t D, float eps, int64_t block, void *workspace,
                        size_t workspace_bytes, const float *state, size_t state_bytes,
                        race_stream stream);

/* The same non-causal pair with V, out, gO and gV as [B][H][T][D] views of any layout (fp32,
 * contiguous last dim, token stride < 2^31) and the probabilities [B*H][T][S] contiguous, stream
 * n = b * H + h. `state` may be null (no kept totals), else as race_nc_op_fwd_keep /
 * race_nc_op_bwd_kept. No counterpart in the reference, whose BatchedACE moves its
 * [M,B,T,H,d_k] values to [M*B*H, T, d_k] and back with torch permute/reshape copies
 * (scaling/benchmark_time.py:116-128,164): for callers whose values keep that layout. */
int race_nc_fwd_view(const float *pK, const float *pQ, race_tensor V, race_tensor out, int64_t B,
                     int64_t H, int64_t T, int64_t S, int64_t D, float eps, int64_t block,
                     void *workspace, size_t workspace_bytes, float *state, size_t state_bytes,
                     race_stream stream);
int race_nc_bwd_view(const float *pK, const float *pQ, race_tensor V, race_tensor gO, float *gpK,
                     float *gpQ, race_tensor gV, int64_t B, int64_t H, int64_t T, int64_t S,
                     int64_t D, float eps, int64_t block, void *workspace, size_t workspace_bytes,
                     const float *state, size_t state_bytes, race_stream stream);

/* ---------------------------------------------------------------- fused layer */
typedef struct {
    int B, Hq, Hkv, T, D; /* q [B][Hq][T][D], k/v [B][Hkv][T][D]; query head h reads kv head h/(Hq/Hkv) */
    int L, K;             /* hash tables and bits, K <= 4 */
    float scale, eps;     /* logits divisor (reference: sqrt(D)) and denominator eps */
    int64_t block;        /* tokens per workgroup, 0: automatic */
} race_qkv_shape;

/* Bytes of the state the forward writes and the backward / final_state read. */
size_t race_qkv_state_bytes(const race_qkv_shape *sh);
/* Bytes of scratch for the forward (backward = 0) or backward (backward = 1). */
size_t race_qkv_scratch_bytes(const race_qkv_shape *sh, int backward);
/* bf16 q, k, v; planes_T fp32 [D][L*K]; out bf16 or fp32 (out_dtype). */
int race_qkv_fwd(const race_qkv_shape *sh, race_tensor q, race_tensor k, race_tensor v,
                 const float *planes_T, race_tensor out, int out_dtype, void *state,
                 size_t state_bytes, void *scratch, size_t scratch_bytes, race_stream stream);
/* go bf16; dq, dk, dv bf16 (overwritten, not accumulated). */
int race_qkv_bwd(const race_qkv_shape *sh, race_tensor q, race_tensor k, race_tensor v,
                 race_tensor go, const float *planes_T, const void *state, size_t state_bytes,
                 race_tensor dq, race_tensor dk, race_tensor dv, void *scratch,
                 size_t scratch_bytes, race_stream stream);
/* race_qkv_bwd without a scratch argument: no counterpart in the reference; for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops). The scratch lives
 * in a static device array of race_static_scratch_bytes() = RACE_STATIC_SCRATCH_BYTES bytes on
 * each GPU the library runs on, held until the process ends. Shapes whose backward scratch
 * (race_qkv_scratch_bytes(sh, 1)) exceeds it fail with RACE_ERR_WORKSPACE (e.g. more than 128
 * buckets at D = 64, whose partial outputs need a workspace); nothing is allocated either way.
 * Calls that overlap on one GPU share the array and race: serialise them (one stream). */
#define RACE_STATIC_SCRATCH_BYTES (32u << 20)
size_t race_static_scratch_bytes(void);
int race_qkv_bwd_static(const race_qkv_shape *sh, race_tensor q, race_tensor k, race_tensor v,
                        race_tensor go, const float *planes_T, const void *state, size_t state_bytes,
                        race_tensor dq, race_tensor dk, race_tensor dv, race_stream stream);
/* Final bucket state after the forward: A [B*Hkv][S], Bs [B*Hkv][S][D] fp32. */
int race_qkv_final_state(const race_qkv_shape *sh, const void *state, size_t state_bytes,
                         float *A, float *Bs, race_stream stream);

/* ---------------------------------------------------------------- decode */
typedef struct {
    int B, Hq, Hkv, D, L, K; /* q [B][Hq][D], k/v [B][Hkv][D]; Hq/Hkv <= 8; D in {64,128} */
    float scale, eps;
} race_decode_shape;

/* One token per sequence: A += pK, Bs += pK v^T (in place, state [B*Hkv][S] /
 * [B*Hkv][S][D] fp32), then out = sum_s pQ Bs / (A + eps). q/k/v/out share dtype. */
int race_decode_step(const race_decode_shape *sh, const void *q, const void *k, const void *v,
                     int dtype, const float *planes_T, float *A, float *Bs, void *out,
                     race_stream stream);

/* ---------------------------------------------------------------- kernel timing */
/* No reference counterpart (the reference times with wall clocks only,
 * scaling/benchmark_time.py:337-351). When enabled, every kernel launch of this
 * library is bracketed by HIP events on its own stream; race_profile_read
 * waits for the recorded events of one kernel and returns its accumulated time
 * and launch count since the last reset. */
enum {
    RACE_PROF_QKV_FWD_TOTALS = 0,
    RACE_PROF_QKV_FWD_READOUT = 1,
    RACE_PROF_QKV_BWD_TOTALS = 2,
    RACE_PROF_QKV_BWD_MAIN = 3,
    RACE_PROF_OP_FWD_TOTALS = 4,
    RACE_PROF_OP_FWD_READOUT = 5,
    RACE_PROF_OP_BWD_TOTALS = 6,
    RACE_PROF_OP_BWD_MAIN = 7,
    RACE_PROF_BLOCK_SCAN = 8,
    RACE_PROF_REDUCE = 9,
    RACE_PROF_SOFTHASH_FWD = 10,
    RACE_PROF_SOFTHASH_BWD = 11,
    RACE_PROF_DECODE = 12,
    RACE_PROF_NC_FWD = 13,
    RACE_PROF_NC_BWD = 14,
    RACE_PROF_KERNELS = 15
};
int race_profile_enable(int on);
int race_profile_read(int kernel, double *total_ms, int64_t *launches);
int race_profile_reset(void);

#ifdef __cplusplus
}
#endif

#endif /* RACE_ATTENTION_H */
