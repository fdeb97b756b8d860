"""Causal RACE modules with the interface of the reference's misc/race.py.

  BatchedACE(d_k, K, L, M, device, share_planes).forward(Khf, Vhf, Qhf)   misc/race.py:26-142
      inputs/outputs [M, B, T, H, d_k]; argument order (K, V, Q); eps 1e-6 and
      scale sqrt(d_k) as misc/race.py:67,110; planes drawn from the global RNG
      (misc/race.py:41,48).
  RACEAttention(d, h, K, L, M, drop, qkv_bias, device, merge)             misc/race.py:144-173
  RACEBlock(cfg, device, merge)                                           misc/race.py:176-206

RACEAttention merges ensembles and heads as the reference does by default
(merge="reference": out_h.mean(0).permute(0,2,1,3).contiguous().view(B,T,-1),
misc/race.py:171). That reinterprets the [B,H,T,d_k] buffer as [B,T,H*d_k]: output row t
holds head floor(t*H/T)'s tokens t*H .. t*H+H-1, so heads and tokens mix and the layer is
not causal. It is reproduced because a checkpoint trained with the reference learned its
output projection on that layout. merge="heads" concatenates the heads of each token
([B,T,H*d_k], causal), the layout a new model wants.

The scan runs on the HIP kernels: bf16 activations (head dim 64/128) take the
fused q/k/v kernels, everything else the HIP soft-hash + fp32 chunked scan.
"""
import itertools
import math

import torch
import torch.nn as nn

from .attention import RaceAttentionFn, fused_supported
from .race_causal_cuda import RaceCausalFn
from .race_common import soft_hash_probs

EPS = 1e-6


def _race_bhtd(Q, K, V, planes_T, protos_T, L, Kb):
    """Causal RACE of [B,H,T,D] inputs with one set of planes; output in Q's dtype."""
    D = Q.shape[-1]
    if fused_supported(Q, K, V, Kb):
        return RaceAttentionFn.apply(Q, K, V, planes_T, L, Kb, math.sqrt(D), EPS, Q.dtype, 0)
    B, H, T, _ = Q.shape
    pK, pQ, V2, N = soft_hash_probs(Q, K, V, planes_T, protos_T, L, Kb, 1, True)
    return RaceCausalFn.apply(pK, pQ, V2, EPS).view(B, H, T, D).to(Q.dtype)


class BatchedACE(nn.Module):
    """Causal BatchedACE with one shared sketch or independent sketches per ensemble."""

    def __init__(self, d_k, K, L, M, device="cpu", share_planes: bool = True):
        super().__init__()
        self.d_k, self.K, self.L, self.M = d_k, K, L, M
        self.R = 1 << K
        self.share_planes = share_planes
        if share_planes:
            planes = torch.randn(L, K, d_k, device=device)
            self.register_buffer("planes_T", planes.view(L * K, d_k).T)
        else:
            planes = torch.randn(M, L, K, d_k, device=device)
            self.register_buffer("planes_T", planes.view(M, L * K, d_k).transpose(1, 2))
        corners = torch.tensor(list(itertools.product([-1.0, 1.0], repeat=K)), device=device)
        self.register_buffer("protos_T", corners.T)

    def forward(self, Khf, Vhf, Qhf):
        M, B, T, H, dk = Khf.shape
        assert M == self.M and dk == self.d_k

        def bhtd(X):  # [M,B,T,H,dk] -> [M*B, H, T, dk] view
            return X.reshape(M * B, T, H, dk).transpose(1, 2)

        if self.share_planes:
            out = _race_bhtd(bhtd(Qhf), bhtd(Khf), bhtd(Vhf), self.planes_T, self.protos_T, self.L, self.K)
            return out.transpose(1, 2).reshape(M, B, T, H, dk)
        outs = []
        for m in range(M):
            q, k, v = (X[m].transpose(1, 2) for X in (Qhf, Khf, Vhf))
            outs.append(_race_bhtd(q, k, v, self.planes_T[m], self.protos_T, self.L, self.K).transpose(1, 2))
        return torch.stack(outs, 0)


class RACEAttention(nn.Module):
    """Multi-head wrapper around BatchedACE (misc/race.py:144-173); `merge` as in the module
    docstring ("reference", the default, or "heads")."""

    def __init__(self, d, h, K, L, M, drop=0.1, qkv_bias=False, device="cpu", merge="reference"):
        super().__init__()
        assert d % h == 0
        if merge not in ("reference", "heads"):
            raise ValueError(f"merge must be 'reference' or 'heads', got {merge!r}")
        self.merge = merge
        self.h, self.d_k, self.M = h, d // h, M
        self.q = nn.Linear(d, d, bias=qkv_bias)
        self.k = nn.Linear(d, d, bias=qkv_bias)
        self.v = nn.Linear(d, d, bias=qkv_bias)
        self.o = nn.Linear(d, d)
        self.drop = nn.Dropout(drop)
        self.ace = BatchedACE(self.d_k, K, L, M, device=device)

    def forward(self, x):
        B, T, _ = x.shape
        Q = self.q(x).view(B, T, self.h, self.d_k)
        K = self.k(x).view(B, T, self.h, self.d_k)
        V = self.v(x).view(B, T, self.h, self.d_k)
        pack = lambda z: z.unsqueeze(0).expand(self.M, -1, -1, -1, -1)  # noqa: E731
        out_h = self.ace(pack(K), pack(V), pack(Q))  # [M, B, T, H, d_k]
        if self.merge == "reference":
            out = out_h.mean(0).permute(0, 2, 1, 3).contiguous().view(B, T, -1)
        else:
            out = out_h.mean(0).contiguous().view(B, T, -1)
        return self.drop(self.o(out))


class RACEBlock(nn.Module):
    """Pre-norm transformer block with RACEAttention (misc/race.py:176-206)."""

    def __init__(self, cfg, device="cpu", merge="reference"):
        super().__init__()
        self.att = RACEAttention(d=cfg["emb_dim"], h=cfg["n_heads"], K=cfg["K"], L=cfg["L"], M=cfg["M"],
                                 drop=cfg["drop_rate"], qkv_bias=cfg["qkv_bias"], device=device, merge=merge)
        self.norm1 = nn.LayerNorm(cfg["emb_dim"])
        self.norm2 = nn.LayerNorm(cfg["emb_dim"])
        self.ff = nn.Sequential(nn.Linear(cfg["emb_dim"], 4 * cfg["emb_dim"]), nn.GELU(),
                                nn.Linear(4 * cfg["emb_dim"], cfg["emb_dim"]))
        self.drop = nn.Dropout(cfg["drop_rate"])

    def forward(self, x):
        h = x
        x = self.drop(self.att(self.norm1(x))) + h
        h = x
        return self.drop(self.ff(self.norm2(x))) + h
