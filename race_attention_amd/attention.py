"""Fused causal RACE attention layer: q, k, v in; out (and dq, dk, dv) out.

One autograd Function over the bf16 fused kernels (race_qkv_fwd / race_qkv_bwd):
the soft-hash of scaling/race_common.py:36-73 and the causal scan of
race_causal_cuda.py:47-69 run inside the same HIP kernels, so the [N,T,S] bucket
probabilities are never written to HBM. The forward saves only q, k, v and the
per-block bucket states; the backward recomputes the probabilities.

Grouped-query attention: q [B,Hq,T,D] with k, v [B,Hkv,T,D]; query head h reads
the bucket state of kv head h // (Hq // Hkv). With Hq == Hkv this is the
reference's multi-head layer.
"""
import math

import torch
from torch.autograd import Function

from . import _lib


def fused_supported(q, k, v, Kbits):
    """True when the bf16 fused kernels cover these inputs."""
    return (q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16
            and q.dim() == 4 and q.shape[-1] in (64, 128) and 1 <= Kbits <= 4
            and q.device.type == "cuda")


def _bf16_rows(t):
    """A [B,H,T,D] bf16 view whose rows the kernels can read as 16-byte vectors."""
    if t.stride(3) != 1 or t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:3]):
        t = t.contiguous()
    return t


def qkv_shape(q, k, L, Kbits, scale, eps, block=0):
    B, Hq, T, D = q.shape
    return _lib.QKVShape(B, Hq, k.shape[1], T, D, L, Kbits, float(scale), float(eps), int(block))


class RaceAttentionFn(Function):
    """out = causal RACE(q, k, v); q [B,Hq,T,D], k/v [B,Hkv,T,D] bf16, planes_T [D, L*K]."""

    @staticmethod
    def forward(ctx, q, k, v, planes_T, L, Kbits, scale, eps, out_dtype, block):
        _lib.require_device(q, k, v, planes_T)
        if not fused_supported(q, k, v, Kbits):
            raise _lib.RaceError("fused RACE needs bf16 q/k/v with head dim 64 or 128 and K <= 4")
        B, Hq, T, D = q.shape
        if k.shape != (B, k.shape[1], T, D) or v.shape != k.shape or Hq % k.shape[1]:
            raise ValueError(f"q {tuple(q.shape)} / k {tuple(k.shape)} / v {tuple(v.shape)} mismatch")
        q, k, v = _bf16_rows(q), _bf16_rows(k), _bf16_rows(v)
        planes = planes_T.detach().float().contiguous()
        if planes.shape != (D, L * Kbits):
            raise ValueError(f"planes_T must be [{D}, {L * Kbits}], got {tuple(planes.shape)}")
        out_dtype = out_dtype or q.dtype
        sh = qkv_shape(q, k, L, Kbits, scale, eps, block)
        lib = _lib.lib()
        state = _lib.workspace(lib.race_qkv_state_bytes(sh), q.device)
        scratch = _lib.workspace(lib.race_qkv_scratch_bytes(sh, 0), q.device)
        out = torch.empty(B, Hq, T, D, dtype=out_dtype, device=q.device)
        qv, _ = _lib.view4(q)
        kv_, _ = _lib.view4(k)
        vv, _ = _lib.view4(v)
        ov, _ = _lib.view4(out)
        _lib.check(lib.race_qkv_fwd(sh, qv, kv_, vv, _lib.ptr(planes), ov, _lib.dtype_code(out_dtype),
                                    _lib.ptr(state), state.numel(), _lib.ptr(scratch), scratch.numel(),
                                    _lib.stream_of(q)), "race_qkv_fwd")
        ctx.save_for_backward(q, k, v, planes, state)
        ctx.cfg = (L, Kbits, float(scale), float(eps), int(block))
        return out

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, planes, state = ctx.saved_tensors
        L, Kbits, scale, eps, block = ctx.cfg
        go = _bf16_rows(grad_out.to(torch.bfloat16))
        sh = qkv_shape(q, k, L, Kbits, scale, eps, block)
        lib = _lib.lib()
        scratch = _lib.workspace(lib.race_qkv_scratch_bytes(sh, 1), q.device)
        dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        dk = torch.empty(k.shape, dtype=k.dtype, device=k.device)
        dv = torch.empty(v.shape, dtype=v.dtype, device=v.device)
        views = [_lib.view4(t)[0] for t in (q, k, v, go, dq, dk, dv)]
        _lib.check(lib.race_qkv_bwd(sh, views[0], views[1], views[2], views[3], _lib.ptr(planes),
                                    _lib.ptr(state), state.numel(), views[4], views[5], views[6],
                                    _lib.ptr(scratch), scratch.numel(), _lib.stream_of(q)), "race_qkv_bwd")
        return dq, dk, dv, None, None, None, None, None, None, None


def race_causal_attention(q, k, v, planes_T, L, Kbits, scale=None, eps=1e-6, out_dtype=None, block=0):
    """Causal RACE attention of bf16 q [B,Hq,T,D], k/v [B,Hkv,T,D] -> [B,Hq,T,D].

    `scale` divides tanh(x . plane) (default sqrt(D) as scaling/race_common.py:46);
    `out_dtype` defaults to q's dtype; `block` sets tokens per workgroup (0: auto).
    """
    if scale is None:
        scale = math.sqrt(q.shape[-1])
    return RaceAttentionFn.apply(q, k, v, planes_T, L, Kbits, scale, eps, out_dtype, block)


def race_causal_attention_with_state(q, k, v, planes_T, L, Kbits, scale=None, eps=1e-6, out_dtype=None):
    """Forward only (no autograd): (out, A [B*Hkv,S], Bs [B*Hkv,S,D]) -- the output and
    the final bucket state (race_prefix_ref's A_final / B_final, race_common.py:88-90),
    which seeds race_attention_amd.decode.RaceDecodeState."""
    _lib.require_device(q, k, v, planes_T)
    if scale is None:
        scale = math.sqrt(q.shape[-1])
    if not fused_supported(q, k, v, Kbits):
        raise _lib.RaceError("fused RACE needs bf16 q/k/v with head dim 64 or 128 and K <= 4")
    q, k, v = _bf16_rows(q), _bf16_rows(k), _bf16_rows(v)
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    planes = planes_T.detach().float().contiguous()
    out_dtype = out_dtype or q.dtype
    sh = qkv_shape(q, k, L, Kbits, scale, eps, 0)
    lib = _lib.lib()
    state = _lib.workspace(lib.race_qkv_state_bytes(sh), q.device)
    scratch = _lib.workspace(lib.race_qkv_scratch_bytes(sh, 0), q.device)
    out = torch.empty(B, Hq, T, D, dtype=out_dtype, device=q.device)
    qv, kv_, vv, ov = (_lib.view4(t)[0] for t in (q, k, v, out))
    _lib.check(lib.race_qkv_fwd(sh, qv, kv_, vv, _lib.ptr(planes), ov, _lib.dtype_code(out_dtype),
                                _lib.ptr(state), state.numel(), _lib.ptr(scratch), scratch.numel(),
                                _lib.stream_of(q)), "race_qkv_fwd")
    S = L << Kbits
    A = torch.empty(B * Hkv, S, dtype=torch.float32, device=q.device)
    Bs = torch.empty(B * Hkv, S, D, dtype=torch.float32, device=q.device)
    _lib.check(lib.race_qkv_final_state(sh, _lib.ptr(state), state.numel(), _lib.ptr(A), _lib.ptr(Bs),
                                        _lib.stream_of(q)), "race_qkv_final_state")
    return out, A, Bs
