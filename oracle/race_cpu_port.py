"""Faithful CPU port of the reference CPU path -- TEST INFRASTRUCTURE / CPU BASELINE.

This is the timed ``cpu_baseline`` (kind "port") of bench.py and a checker in
tests/. It restates, on torch CPU tensors:

  soft_hash_probs_fp32  scaling/race_common.py:36-73 in fp32 torch ops (matmul,
                        tanh, /sqrt(D), @protos, fp32 softmax) exactly as the
                        reference runs on the CPU
  RaceCausalCPUFn       scaling/race_causal_cpu.py:33-72: the x S flatten of
                        probsK and V, the fp64-accumulating prefix-mean kernel
                        (C restatement of kernels/cpu/race_pref.cpp in
                        liborace.so, OpenMP over the N*S streams), the einsum
                        readout, and the exact backward through
                        race_prefix_mean_flat_bw
  race_layer_cpu        the module path: soft-hash + RaceCausalCPUFn + mean over M

Its memory is O(N*S*T*D), as in the reference (race_causal_cpu.py:33-38,51-53),
which is what bounds the CPU path's maximum context.
"""
import math

import torch
from torch.autograd import Function

from . import oracle_c


def soft_hash_probs_fp32(Q, K, V, planes_T, protos_T, L, Kbits, M=1):
    """race_common.py:36-73 (shared planes) on the CPU in the inputs' dtype."""
    B, H, T, D = Q.shape
    R = protos_T.shape[1]
    scale = math.sqrt(D)
    N = M * B * H

    def pack(Z):
        return Z.unsqueeze(0).expand(M, -1, -1, -1, -1).reshape(N, T, D)

    Km, Qm, Vm = pack(K), pack(Q), pack(V)
    pT = planes_T.to(Qm.dtype)
    prT = protos_T.to(Qm.dtype)
    lk = ((Km @ pT).view(N, T, L, Kbits).tanh() / scale) @ prT
    lq = ((Qm @ pT).view(N, T, L, Kbits).tanh() / scale) @ prT
    pK = torch.softmax(lk.float(), dim=-1).reshape(N, T, L * R)
    pQ = torch.softmax(lq.float(), dim=-1).reshape(N, T, L * R)
    return pK, pQ, Vm, N


def _flatten(probsK, V2):
    """race_causal_cpu.py:33-38: [(n,s), t] weights and V copied S times."""
    N, T, S = probsK.shape
    D = V2.shape[2]
    pk_flat = probsK.permute(0, 2, 1).reshape(N * S, T).contiguous()
    v_flat = V2.unsqueeze(1).expand(N, S, T, D).reshape(N * S, T, D).contiguous()
    return pk_flat, v_flat, N, T, S, D


class RaceCausalCPUFn(Function):
    """race_causal_cpu.py:41-72 -- same (probsK, probsQ, V2, eps) signature as RaceCausalFn."""

    @staticmethod
    def forward(ctx, probsK, probsQ, V2, eps):
        probsK = probsK.contiguous().float()
        probsQ = probsQ.contiguous().float()
        V2 = V2.contiguous().float()
        pk_flat, v_flat, N, T, S, D = _flatten(probsK, V2)
        E = oracle_c.prefix_mean_flat(pk_flat, v_flat, eps).view(N, S, T, D)
        out = torch.einsum("nts,nstd->ntd", probsQ, E)
        ctx.save_for_backward(pk_flat, v_flat, probsQ, E)
        ctx.eps = float(eps)
        ctx.shape = (N, T, S, D)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        pk_flat, v_flat, probsQ, E = ctx.saved_tensors
        N, T, S, D = ctx.shape
        grad_out = grad_out.contiguous().float()
        g_pq = torch.einsum("ntd,nstd->nts", grad_out, E).contiguous()
        gE = torch.einsum("nts,ntd->nstd", probsQ, grad_out).reshape(N * S, T, D).contiguous()
        gW, gV = oracle_c.prefix_mean_flat_bw(pk_flat, v_flat, gE, ctx.eps)
        g_pk = gW.view(N, S, T).permute(0, 2, 1).reshape(N, T, S).contiguous()
        g_v = gV.view(N, S, T, D).sum(dim=1).contiguous()
        return g_pk, g_pq, g_v, None


def race_layer_cpu(Q, K, V, planes_T, protos_T, L, Kbits, M=1, eps=1e-6):
    """One RACE layer forward on the CPU (soft-hash + RaceCausalCPUFn + mean over M)."""
    B, H, T, D = Q.shape
    pK, pQ, V2, N = soft_hash_probs_fp32(Q, K, V, planes_T, protos_T, L, Kbits, M)
    out = RaceCausalCPUFn.apply(pK, pQ, V2, eps)
    return out.view(M, B, H, T, D).mean(dim=0)
