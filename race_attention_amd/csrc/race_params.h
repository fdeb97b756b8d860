// Kernel parameter blocks shared by the HIP kernels and the host dispatch code.
#pragma once
#include <stdint.h>

namespace race {

// A [B][H][T][D] tensor view with contiguous last dim (element strides).
struct View {
    const void *p;
    int64_t sb, sh, st;
};

// An output view: like View, plus the element stride between s-tile partials
// (0 when the kernel writes the final tensor) and the element type.
struct OutView {
    void *p;
    int64_t sb, sh, st;
    int64_t tile;   // element offset added per s-tile (partial-sum buffers)
    int f32;        // 1: float32 elements, 0: bfloat16 elements
    // Bucket tiles launched one after another (fused kernels): a non-null acc holds the fp32 sum
    // of the earlier tiles' contributions ([B][H][T][D] with its own element strides), added to
    // this tile's before the store; stage_f32 asks for the kernel variant that stages rows in
    // fp32, so that the sum is rounded once, when the last tile writes it.
    const float *acc;
    int64_t acc_sb, acc_sh, acc_st;
    int stage_f32;
};

// One launch of the chunked causal scan.
//   stream z:  op mode   z = n (one of N independent [T,S]/[T,D] streams)
//              qkv mode  z = b * Hkv + hk (one kv head; query heads hk*G .. hk*G+G-1)
//   grid:      (NB blocks along T, n_st bucket tiles, Z streams)
struct ScanParams {
    int T, S, D, L, K, R;  // tokens, buckets S = L*R, head dim, tables, bits, 2^K
    int G, Hkv;            // query heads per kv head, kv heads (qkv mode)
    int CB, NB;            // tokens per block, blocks
    int n_st, S_pad;       // bucket tiles per stream, n_st * tile
    int st_base;           // bucket tile of grid row blockIdx.y = 0 (tiles launched one at a time)
    int DPw;               // padded head dim used by the state workspaces
    float eps, scale, inv_scale;
    // qkv mode (bf16 activations; planes_T fp32 [D][L*K], shared by all heads)
    View q, k, v, go;
    OutView out, dq, dk, dv;
    const float *planes;
    // op mode (fp32): probabilities [N][T][S], values/grads rows of D floats. Stream z reads its
    // V / gO rows as a [Z / zH][zH][T][D] view: row t of z at (z / zH) sb + (z % zH) sh + t st,
    // strides in v / go (their p unused); contiguous [N][T][D] is zH = 1, sb = T D, st = D
    const float *pK, *pQ, *V, *gO;
    int zH;
    float *gpK, *gpQ;
    // workspaces: block states [Z][NB+1][S_pad][DPw] and [Z][NB+1][S_pad]
    float *wsB, *wsA;    // forward: prefix (A, B) at each block start; slot NB = final
    float *ws2B, *ws2A;  // backward: suffix sums (of W^T go, gA) from each block's start
    // generic backward kernels: low parts of the same suffix sums (ws2 + ws3 = a double-float)
    float *ws3B, *ws3A;
    // op mode only: 1 = unnormalised causal linear attention, W = pQ (no 1/(A+eps), gA = 0)
    int linear;
};

}  // namespace race
