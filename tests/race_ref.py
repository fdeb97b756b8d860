"""fp64 references for the GPU tests, built from the pinned oracle (oracle/).

oracle_op      fp64 streaming C forward/backward of the op-level scan
oracle_layer   fp64 soft-hash (torch autograd) + fp64 streaming C scan, chained:
               out, dq, dk, dv for q [B,Hq,T,D], k/v [B,Hkv,T,D] (GQA by repeat),
               with memory O(T*S) so long sequences stay checkable.
"""
import math

import torch

from oracle import oracle_c
from oracle import race_oracle as orc

F64 = torch.float64


def relerr(got, ref):
    return orc.relerr(got, ref)


def check(name, got, ref, tol, abs_floor=2e-5):
    """The reference's pass rule (scaling/test_kernels.py:38-51): relerr <= tol, or a
    tight absolute floor for genuinely near-zero references."""
    re = orc.relerr(got, ref)
    ma = orc.maxabs(got, ref)
    assert re <= tol or ma <= abs_floor, f"{name}: relerr {re:.3e} > {tol:.0e} (maxabs {ma:.3e})"
    return re


def make_probs(N, T, L, R, D, seed, dist="softmax"):
    """scaling/test_kernels.py:54-66 input distributions, fp64 on the CPU."""
    g = torch.Generator().manual_seed(seed)
    if dist == "softmax":
        pk = torch.softmax(torch.randn(N, T, L, R, generator=g, dtype=F64), -1).reshape(N, T, L * R)
        pq = torch.softmax(torch.randn(N, T, L, R, generator=g, dtype=F64), -1).reshape(N, T, L * R)
    else:
        pk = torch.rand(N, T, L * R, generator=g, dtype=F64)
        pq = torch.rand(N, T, L * R, generator=g, dtype=F64)
    v = torch.randn(N, T, D, generator=g, dtype=F64)
    go = torch.randn(N, T, D, generator=g, dtype=F64)
    return pk, pq, v, go


def oracle_op(pk, pq, v, go, eps):
    out, A, B = oracle_c.race_fwd(pk, pq, v, eps)
    gpk, gpq, gv = oracle_c.race_bwd(pk, pq, v, go, eps)
    return out, gpk, gpq, gv, A, B


def oracle_layer(q, k, v, planes_T, L, Kb, scale, eps, go=None):
    """fp64 out (and dq, dk, dv if go is given). Inputs may be bf16: they are taken
    at their exact values; planes are taken as given (round them to bf16 first to
    match a bf16 run, as the reference does at race_common.py:54)."""
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    rep = Hq // Hkv
    q64 = q.detach().to("cpu", F64).requires_grad_(go is not None)
    k64 = k.detach().to("cpu", F64).requires_grad_(go is not None)
    v64 = v.detach().to("cpu", F64).requires_grad_(go is not None)
    kr = k64.repeat_interleave(rep, dim=1)
    vr = v64.repeat_interleave(rep, dim=1)
    _, protos = orc.build_planes_protos(D, Kb, L)
    pK, pQ, V2, N = orc.soft_hash_probs(q64, kr, vr, planes_T.detach().cpu().to(F64), protos, L, Kb,
                                        scale=scale)
    out, _, _ = oracle_c.race_fwd(pK.detach(), pQ.detach(), V2.detach(), eps)
    out = out.view(B, Hq, T, D)
    if go is None:
        return out
    g64 = go.detach().to("cpu", F64).reshape(N, T, D)
    gpk, gpq, gv = oracle_c.race_bwd(pK.detach(), pQ.detach(), V2.detach(), g64, eps)
    torch.autograd.backward([pK, pQ, V2], [gpk, gpq, gv])
    return out, q64.grad, k64.grad, v64.grad


def bf16_planes(planes_T):
    return planes_T.to(torch.bfloat16).float()


def default_scale(D):
    return math.sqrt(D)
