"""MI355X-native causal RACE attention (hand-written HIP kernels for gfx950).

Public surface (mirrors sahiljoshi515/RACE_Attention):
  build_planes_protos, soft_hash_probs,
  race_prefix_ref                                (scaling/race_common.py)
  RaceCausalFn, RaceCausalCuda, race_cuda_fused,
  race_fused_fwd, race_backward, fwd_chunk       (scaling/race_causal_cuda.py, kernels/gpu)
  RaceCumsumCausal                               (scaling/race_torch_cumsum.py)
  BatchedACE, RACEAttention, RACEBlock           (misc/race.py)
plus the fused layer race_causal_attention (q, k, v in; GQA) and RaceDecodeState
(single-token decode on the carried bucket state).
"""
from .attention import RaceAttentionFn, race_causal_attention, race_causal_attention_with_state
from .decode import RaceDecodeState
from .race import BatchedACE, RACEAttention, RACEBlock
from .race_causal_cuda import (RaceCausalCuda, RaceCausalFn, fwd_chunk, race_backward, race_cuda_fused,
                               race_fused_fwd)
from .race_common import build_planes_protos, race_prefix_ref, soft_hash_probs
from .race_torch_cumsum import RaceCumsumCausal

__all__ = [
    "build_planes_protos", "soft_hash_probs", "race_prefix_ref", "RaceCausalFn", "RaceCausalCuda", "race_cuda_fused",
    "race_fused_fwd", "race_backward", "fwd_chunk", "RaceCumsumCausal", "BatchedACE", "RACEAttention",
    "RACEBlock", "RaceAttentionFn", "race_causal_attention", "race_causal_attention_with_state",
    "RaceDecodeState",
]
