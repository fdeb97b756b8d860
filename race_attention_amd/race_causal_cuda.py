"""Causal RACE attention on MI355X with the reference's interface
(scaling/race_causal_cuda.py).

  race_fused_fwd(probsK, probsQ, V2, eps, chunk) -> out        kernels/gpu/forward_kernel.cu:110
  race_backward(probsK, probsQ, V2, grad_out, eps, chunk)      kernels/gpu/backward_kernels.cu:174
      -> [gradProbsK, gradProbsQ, gradV]
  fwd_chunk(T)                                                 race_causal_cuda.py:33-44
  RaceCausalFn.apply(probsK, probsQ, V2, eps) -> out [N,T,D]   race_causal_cuda.py:47-69
  race_cuda_fused(probsK, probsQ, V2, eps)                     race_causal_cuda.py:72-73
  _ext() -> object with race_fused_fwd / race_backward         race_causal_cuda.py:26-30
  RaceCausalCuda(d_k, Kbits, L, M, device, share_planes, eps, seed)   race_causal_cuda.py:76-102

The op-level functions run the fp32 chunked-scan HIP kernels (race_op_fwd /
race_op_bwd). RaceCausalCuda runs the fused bf16 q/k/v kernels when its inputs
are bf16 with a supported head dim (the soft-hash happens inside the scan and
the [N,T,S] probabilities never reach HBM); otherwise it composes the HIP
soft-hash with RaceCausalFn exactly as the reference does. Its output is fp32
[B,H,T,D] in both cases, as the reference's.
"""
import math

import torch
import torch.nn as nn
from torch.autograd import Function

from . import _lib
from .attention import RaceAttentionFn, fused_supported
from .race_common import build_planes_protos, soft_hash_probs


def fwd_chunk(T):
    """The reference's chunk heuristic (race_causal_cuda.py:33-44), kept for callers
    that pass it on; the HIP kernels choose their own block size when given 0 and
    their results do not depend on it beyond fp32 rounding."""
    if T <= 4096:
        return int(T)
    e = int(math.ceil(math.log2(max(1.0, T / 48.0))))
    e = max(11, min(16, e))
    return min(1 << e, int(T))


def _op_inputs(probsK, probsQ, V2):
    _lib.require_device(probsK, probsQ, V2)
    if probsK.dim() != 3 or probsQ.shape != probsK.shape or V2.dim() != 3 or V2.shape[:2] != probsK.shape[:2]:
        raise ValueError("shapes must be probsK/probsQ [N,T,S] and V2 [N,T,D], got "
                         f"{tuple(probsK.shape)}, {tuple(probsQ.shape)}, {tuple(V2.shape)}")
    return probsK.contiguous().float(), probsQ.contiguous().float(), V2.contiguous().float()


def state_buffer(nbytes, device, what):
    """A 256-byte aligned device buffer of `nbytes` for a kept forward state; nbytes = 0 means the
    library rejected the geometry, whose reason is raised."""
    if nbytes == 0:
        raise _lib.RaceError(f"{what}: {_lib.lib().race_last_error().decode(errors='replace')}")
    return torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=device)


def op_state(probsK, V2, chunk=0):
    """A buffer for the forward block states that race_fused_fwd(..., state=) keeps for
    race_backward(..., state=)."""
    N, T, S = probsK.shape
    n = _lib.lib().race_op_state_bytes(N, T, S, V2.shape[2], max(int(chunk), 0))
    return state_buffer(n, probsK.device, "race_op_state_bytes")


def state_arg(state):
    """(pointer, size in bytes) of a kept-state buffer, as the *_keep / *_kept entry points take them."""
    return _lib.ptr(state), state.numel() * state.element_size()


def race_fused_fwd(probsK, probsQ, V2, eps, chunk=0, state=None):
    """out[N,T,D] fp32 = causal RACE(probsK, probsQ, V2) (forward_kernel.cu:110-137).
    `chunk` is the tokens per workgroup block (<= 0: automatic). With `state` (op_state), the
    scanned forward block states are left there for race_backward."""
    pK, pQ, V = _op_inputs(probsK, probsQ, V2)
    N, T, S = pK.shape
    D = V.shape[2]
    block = max(int(chunk), 0)
    L = _lib.lib()
    ws = _lib.workspace(L.race_op_workspace_bytes(N, T, S, D, block, 0), pK.device)
    out = torch.empty(N, T, D, dtype=torch.float32, device=pK.device)
    args = (_lib.ptr(pK), _lib.ptr(pQ), _lib.ptr(V), _lib.ptr(out), N, T, S, D, float(eps), block, _lib.ptr(ws),
            ws.numel())
    if state is None:
        _lib.check(L.race_op_fwd(*args, _lib.stream_of(pK)), "race_op_fwd")
    else:
        _lib.check(L.race_op_fwd_keep(*args, *state_arg(state), _lib.stream_of(pK)), "race_op_fwd_keep")
    return out


def race_backward(probsK, probsQ, V2, grad_out, eps, chunk=0, state=None):
    """[gradProbsK, gradProbsQ, gradV] (backward_kernels.cu:174-215), exact. With `state` from
    race_fused_fwd(..., state=) on the same inputs and chunk, the forward block states are read
    from it instead of recomputed."""
    pK, pQ, V = _op_inputs(probsK, probsQ, V2)
    _lib.require_device(grad_out)
    gO = grad_out.contiguous().float()
    N, T, S = pK.shape
    D = V.shape[2]
    block = max(int(chunk), 0)
    L = _lib.lib()
    ws = _lib.workspace(L.race_op_workspace_bytes(N, T, S, D, block, 1), pK.device)
    gpk = torch.empty_like(pK)
    gpq = torch.empty_like(pQ)
    gv = torch.empty_like(V)
    args = (_lib.ptr(pK), _lib.ptr(pQ), _lib.ptr(V), _lib.ptr(gO), _lib.ptr(gpk), _lib.ptr(gpq), _lib.ptr(gv), N, T,
            S, D, float(eps), block, _lib.ptr(ws), ws.numel())
    if state is None:
        _lib.check(L.race_op_bwd(*args, _lib.stream_of(pK)), "race_op_bwd")
    else:
        _lib.check(L.race_op_bwd_kept(*args, *state_arg(state), _lib.stream_of(pK)), "race_op_bwd_kept")
    return [gpk, gpq, gv]


class RaceCausalFn(Function):
    """out = causal RACE(probsK, probsQ, V2); exact grads w.r.t. probsK/probsQ/V2."""

    @staticmethod
    def forward(ctx, probsK, probsQ, V2, eps):
        pK, pQ, V = _op_inputs(probsK, probsQ, V2)
        # the forward block states stay in `state` for the backward (not recomputed there)
        state = op_state(pK, V)
        out = race_fused_fwd(pK, pQ, V, eps, 0, state=state)
        ctx.save_for_backward(pK, pQ, V, state)
        ctx.eps = float(eps)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        pK, pQ, V, state = ctx.saved_tensors
        gpk, gpq, gv = race_backward(pK, pQ, V, grad_out, ctx.eps, 0, state=state)
        return gpk, gpq, gv, None


def race_cuda_fused(probsK, probsQ, V2, eps=1e-6):
    return RaceCausalFn.apply(probsK, probsQ, V2, eps)


class _Ext:
    """The extension object the reference's _ext() returns (race_causal_cuda.py:26-30), whose
    bound ops (race_cuda_binding.cpp:12-23) its tests call directly (scaling/test_kernels.py:87-89):
    race_fused_fwd(pK, pQ, V2, eps, chunk) and race_backward(pK, pQ, V2, gO, eps, chunk), here the
    HIP op kernels through the C ABI."""
    race_fused_fwd = staticmethod(race_fused_fwd)
    race_backward = staticmethod(race_backward)


_EXT = _Ext()


def _ext():
    """The library's op entry points under the reference's accessor name (loads librace_amd.so;
    raises if it is missing: there is no fallback)."""
    _lib.lib()
    return _EXT


class RaceCausalCuda(nn.Module):
    """Causal RACE over Q,K,V [B,H,T,D] -> [B,H,T,D] fp32 (race_causal_cuda.py:76-102)."""

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
        if self.share_planes and fused_supported(Q, K, V, self.Kbits):
            # the M ensemble copies share the planes, so their mean is one copy
            return RaceAttentionFn.apply(Q, K, V, self.planes_T, self.L, self.Kbits, math.sqrt(D),
                                         self.eps, torch.float32, 0)
        probsK, probsQ, V2, N = soft_hash_probs(Q, K, V, self.planes_T, self.protos_T,
                                                self.L, self.Kbits, self.M, self.share_planes)
        out_NTD = RaceCausalFn.apply(probsK, probsQ, V2, self.eps)
        return out_NTD.view(self.M, B, H, T, D).mean(dim=0)
