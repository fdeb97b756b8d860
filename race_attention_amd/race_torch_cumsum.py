"""RaceCumsumCausal -- the reference's pure-PyTorch comparison module
(scaling/race_torch_cumsum.py:14-36), kept for API parity.

It materialises the [N,T,S,D] prefix sums with torch.cumsum (race_common.py:84-87)
and therefore runs out of memory at long T; that limitation is its purpose as a
baseline next to RaceCausalCuda. It is a separate module, not a fallback: no HIP
path in this package calls it. Its soft-hash is the HIP soft_hash_probs.
"""
import torch.nn as nn

from .race_common import build_planes_protos, race_prefix_ref, soft_hash_probs


class RaceCumsumCausal(nn.Module):
    def __init__(self, d_k, Kbits, L, M, device="cuda", share_planes=True, eps=1e-6, seed=0):
        super().__init__()
        self.d_k, self.Kbits, self.L, self.M = d_k, Kbits, L, M
        self.share_planes = share_planes
        self.eps = eps
        planes_T, protos_T = build_planes_protos(d_k, Kbits, L, M, device=device,
                                                 share_planes=share_planes, seed=seed)
        self.register_buffer("planes_T", planes_T)
        self.register_buffer("protos_T", protos_T)

    def forward(self, Q, K, V):
        B, H, T, D = Q.shape
        probsK, probsQ, V2, N = soft_hash_probs(Q, K, V, self.planes_T, self.protos_T,
                                                self.L, self.Kbits, self.M, self.share_planes)
        out_NTD, _, _ = race_prefix_ref(probsK, probsQ, V2.float(), self.eps)
        return out_NTD.view(self.M, B, H, T, D).mean(dim=0)
