"""Causal linear attention (Katharopoulos et al.), the reference's comparison kernel
(kernels/cpu/linear_pref.cpp:87-213, bound in kernels/cpu/race_ext.py:57-66):

  causal_dot_product(Q, K, V, out):   out_l = Q_l . sum_{s<=l} K_s (x) V_s
  causal_dot_backward(Q, K, V, g, gQ, gK, gV)

Q, K [N,H,L,E], V [N,H,L,M] fp32. On MI355X this is the causal RACE scan with the
1/(A+eps) normalisation removed (race_causal_dot_product / race_causal_dot_backward):
K plays the bucket probabilities of keys, Q those of queries, E the bucket count.
"""
import torch
from torch.autograd import Function

from . import _lib
from .race_causal_cuda import state_arg, state_buffer


def _flat(x):
    N, H, L, F = x.shape
    return x.detach().float().contiguous().view(N * H, L, F)


def _dest(t, inputs):
    """The [N*H, L, F] fp32 buffer a kernel writes for output `t`: `t` itself when it is contiguous
    fp32 and shares no storage with an input (the kernels read their inputs in several passes),
    otherwise a temporary that the caller copies into `t`."""
    N, H, L, F = t.shape
    st = t.untyped_storage().data_ptr()
    if t.dtype == torch.float32 and t.is_contiguous() and all(st != x.untyped_storage().data_ptr() for x in inputs):
        return t.view(N * H, L, F), False
    return torch.empty(N * H, L, F, dtype=torch.float32, device=t.device), True


def linear_state(queries, values):
    """A buffer for the block states that causal_dot_product(..., state=) keeps for
    causal_dot_backward(..., state=)."""
    N, H, L, E = queries.shape
    n = _lib.lib().race_op_state_bytes(N * H, L, E, values.shape[3], 0)
    return state_buffer(n, queries.device, "race_op_state_bytes")


def causal_dot_product(queries, keys, values, product, state=None):
    """Writes out = causal linear attention into `product` [N,H,L,M] (as the reference). With
    `state` (linear_state), the block states are left there for causal_dot_backward."""
    _lib.require_device(queries, keys, values, product)
    N, H, L, E = queries.shape
    M = values.shape[3]
    if keys.shape != queries.shape or values.shape[:3] != queries.shape[:3] or product.shape != values.shape:
        raise ValueError("expected Q, K [N,H,L,E], V and product [N,H,L,M]")
    Q, K, V = _flat(queries), _flat(keys), _flat(values)
    out, copy_out = _dest(product, (queries, keys, values, Q, K, V))
    lib = _lib.lib()
    ws = _lib.workspace(lib.race_op_workspace_bytes(N * H, L, E, M, 0, 0), Q.device)
    args = (_lib.ptr(Q), _lib.ptr(K), _lib.ptr(V), _lib.ptr(out), N * H, L, E, M, 0, _lib.ptr(ws), ws.numel())
    if state is None:
        _lib.check(lib.race_causal_dot_product(*args, _lib.stream_of(Q)), "race_causal_dot_product")
    else:
        _lib.check(lib.race_causal_dot_product_keep(*args, *state_arg(state), _lib.stream_of(Q)),
                   "race_causal_dot_product_keep")
    if copy_out:
        product.copy_(out.view(N, H, L, M))
    return product


def causal_dot_backward(queries, keys, values, grad_out, grad_queries, grad_keys, grad_values, state=None):
    """Writes the gradients of causal_dot_product into grad_queries / grad_keys / grad_values;
    with `state` from causal_dot_product(..., state=) on the same inputs, the forward block
    states are read from it instead of recomputed."""
    _lib.require_device(queries, keys, values, grad_out)
    N, H, L, E = queries.shape
    M = values.shape[3]
    Q, K, V, G = _flat(queries), _flat(keys), _flat(values), _flat(grad_out)
    ins = (queries, keys, values, grad_out, Q, K, V, G)
    (gQ, cq), (gK, ck), (gV, cv) = _dest(grad_queries, ins), _dest(grad_keys, ins), _dest(grad_values, ins)
    lib = _lib.lib()
    ws = _lib.workspace(lib.race_op_workspace_bytes(N * H, L, E, M, 0, 1), Q.device)
    args = (_lib.ptr(Q), _lib.ptr(K), _lib.ptr(V), _lib.ptr(G), _lib.ptr(gQ), _lib.ptr(gK), _lib.ptr(gV), N * H, L, E,
            M, 0, _lib.ptr(ws), ws.numel())
    if state is None:
        _lib.check(lib.race_causal_dot_backward(*args, _lib.stream_of(Q)), "race_causal_dot_backward")
    else:
        _lib.check(lib.race_causal_dot_backward_kept(*args, *state_arg(state), _lib.stream_of(Q)),
                   "race_causal_dot_backward_kept")
    for dst, buf, cp in ((grad_queries, gQ, cq), (grad_keys, gK, ck), (grad_values, gV, cv)):
        if cp:
            dst.copy_(buf.view(dst.shape))


class CausalLinearFn(Function):
    """Autograd wrapper (the reference test's LinFn, kernels/cpu/test_cpu_kernels.py:110-124)."""

    @staticmethod
    def forward(ctx, Q, K, V):
        out = torch.empty(Q.shape[0], Q.shape[1], Q.shape[2], V.shape[3], dtype=torch.float32, device=Q.device)
        state = linear_state(Q, V)  # the block states stay there for the backward
        causal_dot_product(Q, K, V, out, state=state)
        ctx.save_for_backward(Q, K, V, state)
        return out

    @staticmethod
    def backward(ctx, g):
        Q, K, V, state = ctx.saved_tensors
        gQ = torch.empty(Q.shape, dtype=torch.float32, device=Q.device)
        gK = torch.empty(K.shape, dtype=torch.float32, device=K.device)
        gV = torch.empty(V.shape, dtype=torch.float32, device=V.device)
        causal_dot_backward(Q, K, V, g, gQ, gK, gV, state=state)
        return gQ.to(Q.dtype), gK.to(K.dtype), gV.to(V.dtype)


def causal_linear_attention(Q, K, V):
    return CausalLinearFn.apply(Q, K, V)
