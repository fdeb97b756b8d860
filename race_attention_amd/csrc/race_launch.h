// Host-side launch interface between the C-ABI layer and the kernel objects.
#pragma once
#include <hip/hip_runtime.h>

#include "race_params.h"

namespace race {

enum ScanKernel { K_FWD_TOTALS = 0, K_FWD_READOUT = 1, K_BWD_TOTALS = 2, K_BWD_MAIN = 3 };

// Tile geometry of one compiled variant.
struct Variant {
    int ST;  // buckets per workgroup tile
    int DP;  // padded head dim
    int C;   // tokens per sub-chunk
    int NW;  // waves per workgroup
};

// bf16 fused q/k/v variants (race_scan_qkv.hip). Returns hipErrorInvalidValue for
// an uncompiled (ST, DP) pair.
hipError_t launch_scan_qkv(ScanKernel k, int ST, int DP, const ScanParams &P, dim3 grid,
                           hipStream_t s);
// fp32 probabilities-in variants (race_scan_op.hip).
hipError_t launch_scan_op(ScanKernel k, int ST, int DP, const ScanParams &P, dim3 grid,
                          hipStream_t s);
bool qkv_variant_exists(int ST, int DP);
// fused bf16 forward kernels specialised on the hash bits (race_fused.hip)
hipError_t launch_fused(ScanKernel k, int ST, int DP, int KB, const ScanParams &P, dim3 grid, hipStream_t s);
bool fused_variant_exists(int ST, int DP, int KB);
constexpr int FUSED_NW_FWD = 4, FUSED_NW_BWD = 8;
bool op_variant_exists(int ST, int DP);
constexpr int QKV_C = 32, QKV_NW = 4;
// fp32 op path: waves per workgroup. 4 for the totals kernels; for the readout and backward main
// kernels 8 at head-dim tiles of 64 and more, whose long sub-chunk phases hide more latency with
// them (at 2^20 (token, head) pairs and D = 64: 1.57 -> 1.05 and 4.81 -> 3.50 ms; D = 128 and
// 256 alike), and 4 at 32, where 8 measured slower
constexpr int OP_C = 16, OP_NW_TOTALS = 4;
constexpr int op_nw_main(int DP) { return DP >= 64 ? 8 : 4; }

// race_common.hip
// scans wsB [Z][NB+1][elemsB] and wsA [Z][NB+1][elemsA] over the block axis in one launch; with
// loB / loA (both or neither) every value is the double-float hi (ws) + lo (lo array, same layout)
hipError_t launch_block_scan(float *wsB, int64_t elemsB, float *wsA, int64_t elemsA, int NB, int Z, int rev,
                             hipStream_t s, float *loB = nullptr, float *loA = nullptr);
// out[i] (view, f32 or bf16) = sum_{st < n_st} part[st * tile + i] over a [B][H][T][D] box
hipError_t launch_reduce_partials(const float *part, int n_st, int64_t tile, const OutView &out,
                                  int B, int H, int T, int D, hipStream_t s);

}  // namespace race
