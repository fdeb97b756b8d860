"""Soft-hash pieces with the reference's interface (scaling/race_common.py).

  build_planes_protos(d_k, Kbits, L, M, device, share_planes, dtype, seed)
      -- scaling/race_common.py:14-33: hyperplanes from a CPU Generator seeded with
         `seed`, so a given seed gives the same planes as the reference.
  soft_hash_probs(Q, K, V, planes_T, protos_T, L, Kbits, M, share_planes)
      -- scaling/race_common.py:36-73, computed by the HIP soft-hash kernel
         (differentiable: the backward is the HIP soft-hash backward).
  race_prefix_ref(probsK, probsQ, V2, eps)
      -- scaling/race_common.py:76-90: the reference's pure-torch cumsum specification of
         the causal scan, (out, A_final, B_final). It materialises [N,T,S,D] and runs out of
         memory at long T, as the reference's does; it is the comparison function the
         reference's callers import (scaling/race_torch_cumsum.py:11, scaling/test_kernels.py:19),
         never a path of the HIP kernels.

The corner prototypes protos_T are accepted for signature compatibility; the
kernel uses the closed form of the softmax over the 2^K corners
(p[r] = prod_k sigmoid(2 c_k(r) u_k)), which is what protos_T encodes.
"""
import itertools
import math

import torch
from torch.autograd import Function

from . import _lib


def build_planes_protos(d_k, Kbits, L, M, device="cuda", share_planes=True,
                        dtype=torch.float32, seed=0):
    """planes_T [d_k, L*Kbits] (or [M, d_k, L*Kbits] unshared), protos_T [Kbits, 2^Kbits]."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    if share_planes:
        planes = torch.randn(L, Kbits, d_k, generator=g)
        planes_T = planes.view(L * Kbits, d_k).T.contiguous()
    else:
        planes = torch.randn(M, L, Kbits, d_k, generator=g)
        planes_T = planes.view(M, L * Kbits, d_k).transpose(1, 2).contiguous()
    planes_T = planes_T.to(device=device, dtype=dtype)
    corners = torch.tensor(list(itertools.product([-1.0, 1.0], repeat=Kbits)), dtype=dtype, device=device)
    protos_T = corners.T.contiguous()
    return planes_T, protos_T


def _hash_shape(X, L, Kbits, M, unshared, scale):
    B, H, T, D = X.shape
    return _lib.HashShape(B, H, T, D, L, Kbits, M, 1 if unshared else 0, float(scale))


class SoftHashFn(Function):
    """probs [Mp*B*H, T, L*2^K] fp32 of X [B,H,T,D] (Mp = M when unshared, else 1)."""

    @staticmethod
    def forward(ctx, X, planes_T, L, Kbits, M, unshared, scale):
        _lib.require_device(X, planes_T)
        B, H, T, D = X.shape
        code = _lib.dtype_code(X.dtype)
        planes = planes_T.detach().float().contiguous()
        xv, Xc = _lib.view4(X)
        Mp = M if unshared else 1
        probs = torch.empty(Mp * B * H, T, L << Kbits, dtype=torch.float32, device=X.device)
        sh = _hash_shape(X, L, Kbits, M, unshared, scale)
        _lib.check(_lib.lib().race_soft_hash_fwd(sh, xv, code, _lib.ptr(planes), _lib.ptr(probs),
                                                 _lib.stream_of(X)), "race_soft_hash_fwd")
        ctx.save_for_backward(Xc, planes)
        ctx.cfg = (L, Kbits, M, unshared, scale)
        return probs

    @staticmethod
    def backward(ctx, gprobs):
        Xc, planes = ctx.saved_tensors
        L, Kbits, M, unshared, scale = ctx.cfg
        B, H, T, D = Xc.shape
        Mp = M if unshared else 1
        g = gprobs.float().contiguous().view(Mp, B * H, T, -1)
        dX = torch.empty(B, H, T, D, dtype=Xc.dtype, device=Xc.device)
        xv, _ = _lib.view4(Xc)
        dv, _ = _lib.view4(dX)
        sh = _hash_shape(Xc, L, Kbits, Mp, unshared, scale)
        _lib.check(_lib.lib().race_soft_hash_bwd(sh, xv, _lib.dtype_code(Xc.dtype), _lib.ptr(planes),
                                                 _lib.ptr(g), dv, _lib.stream_of(Xc)), "race_soft_hash_bwd")
        return dX, None, None, None, None, None, None


def soft_hash_probs(Q, K, V, planes_T, protos_T, L, Kbits, M, share_planes=True, scale=None):
    """(probsK, probsQ, V2, N) as scaling/race_common.py:36-73.

    probsK/probsQ [N,T,S] fp32 with N ordered (M,B,H) and S = L*2^K (L-outer);
    V2 [N,T,D] in V's dtype. `scale` (default sqrt(D), as the reference) divides
    the tanh'd projections.
    """
    B, H, T, D = Q.shape
    R = protos_T.shape[1]
    if R != (1 << Kbits):
        raise ValueError(f"protos_T has {R} corners, expected 2^{Kbits}")
    if scale is None:
        scale = math.sqrt(D)
    N = M * B * H
    unshared = not share_planes
    pK = SoftHashFn.apply(K, planes_T, L, Kbits, M, unshared, scale)
    pQ = SoftHashFn.apply(Q, planes_T, L, Kbits, M, unshared, scale)
    if not unshared and M > 1:
        pK = pK.unsqueeze(0).expand(M, -1, -1, -1).reshape(N, T, L * R)
        pQ = pQ.unsqueeze(0).expand(M, -1, -1, -1).reshape(N, T, L * R)
    V2 = V.unsqueeze(0).expand(M, -1, -1, -1, -1).reshape(N, T, D)
    return pK, pQ, V2, N


def race_prefix_ref(probsK, probsQ, V2, eps=1e-6):
    """(out [N,T,D], A_final [N,S], B_final [N,S,D]) of probsK, probsQ [N,T,S], V2 [N,T,D] by
    materialised torch cumsums, on the tensors' own device (scaling/race_common.py:76-90)."""
    A_pref = probsK.cumsum(dim=1)
    B_pref = (probsK.unsqueeze(-1) * V2.unsqueeze(2)).cumsum(dim=1)
    E_pref = B_pref / (A_pref.unsqueeze(-1) + eps)
    out = (probsQ.unsqueeze(-1) * E_pref).sum(dim=2)
    return out, A_pref[:, -1].contiguous(), B_pref[:, -1].contiguous()
