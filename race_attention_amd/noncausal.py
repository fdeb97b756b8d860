"""Non-causal RACE (BatchedACE of scaling/benchmark_time.py:77-176) on the MI355X kernels.

The reference computes, per stream n = (m, b, h), the whole-sequence bucket summaries
A = sum_t pK, B = pK^T V, E = B / (A + eps) and reads them out with out = pQ E
(benchmark_time.py:139-160), through torch bmm in fp32, with a learnable softmax
temperature scale = exp(logit_temp).clamp(1e-2, 10) (benchmark_time.py:104,111).

Here the summaries are the per-block totals of the causal scan machinery (one totals
kernel and the block scan, whose last slot is the whole-sequence sum) and the readout
and its backward are HIP kernels (race_nc_op_fwd / race_nc_op_bwd; race_nc_fwd_view /
race_nc_bwd_view with the values in BatchedACE's [M,B,T,H,d_k] layout). The soft-hash runs
in the HIP soft-hash kernels; with a learnable temperature its backward also returns
d loss / d scale, reduced on the device from per-workgroup partial sums with the scale
read from device memory (race_soft_hash_fwd_dscale / race_soft_hash_bwd_dscale).
"""
import itertools

import torch
import torch.nn as nn
from torch.autograd import Function

from . import _lib
from .race_causal_cuda import _op_inputs, op_state, state_arg, state_buffer
from .race_common import _hash_shape


def race_nc_fwd(probsK, probsQ, V2, eps, block=0, state=None):
    """With `state` (race_causal_cuda.op_state), the whole-sequence totals are left there for
    race_nc_bwd."""
    pK, pQ, V = _op_inputs(probsK, probsQ, V2)
    N, T, S = pK.shape
    D = V.shape[2]
    lib = _lib.lib()
    ws = _lib.workspace(lib.race_nc_op_workspace_bytes(N, T, S, D, block, 0), pK.device)
    out = torch.empty(N, T, D, dtype=torch.float32, device=pK.device)
    args = (_lib.ptr(pK), _lib.ptr(pQ), _lib.ptr(V), _lib.ptr(out), N, T, S, D, float(eps), block, _lib.ptr(ws),
            ws.numel())
    if state is None:
        _lib.check(lib.race_nc_op_fwd(*args, _lib.stream_of(pK)), "race_nc_op_fwd")
    else:
        _lib.check(lib.race_nc_op_fwd_keep(*args, *state_arg(state), _lib.stream_of(pK)), "race_nc_op_fwd_keep")
    return out


def race_nc_bwd(probsK, probsQ, V2, grad_out, eps, block=0, state=None):
    pK, pQ, V = _op_inputs(probsK, probsQ, V2)
    N, T, S = pK.shape
    D = V.shape[2]
    gO = grad_out.float().contiguous()
    lib = _lib.lib()
    ws = _lib.workspace(lib.race_nc_op_workspace_bytes(N, T, S, D, block, 1), pK.device)
    gpK, gpQ, gV = torch.empty_like(pK), torch.empty_like(pQ), torch.empty_like(V)
    args = (_lib.ptr(pK), _lib.ptr(pQ), _lib.ptr(V), _lib.ptr(gO), _lib.ptr(gpK), _lib.ptr(gpQ), _lib.ptr(gV), N, T,
            S, D, float(eps), block, _lib.ptr(ws), ws.numel())
    if state is None:
        _lib.check(lib.race_nc_op_bwd(*args, _lib.stream_of(pK)), "race_nc_op_bwd")
    else:
        _lib.check(lib.race_nc_op_bwd_kept(*args, *state_arg(state), _lib.stream_of(pK)), "race_nc_op_bwd_kept")
    return gpK, gpQ, gV


class RaceNonCausalFn(Function):
    """out [N,T,D] fp32 = pQ (pK^T V) / (sum_t pK + eps) for probsK/probsQ [N,T,S], V2 [N,T,D]."""

    @staticmethod
    def forward(ctx, probsK, probsQ, V2, eps):
        # contiguous fp32 once, saved as such (a strided V2 view is not copied again in the backward)
        pK, pQ, V = _op_inputs(probsK, probsQ, V2)
        state = op_state(pK, V)  # the totals stay there for the backward
        out = race_nc_fwd(pK, pQ, V, eps, state=state)
        ctx.save_for_backward(pK, pQ, V, state)
        ctx.v_dtype = V2.dtype
        ctx.eps = float(eps)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        pK, pQ, V, state = ctx.saved_tensors
        gpK, gpQ, gV = race_nc_bwd(pK, pQ, V, grad_out, ctx.eps, state=state)
        return gpK, gpQ, gV.to(ctx.v_dtype), None


def _bhtd(X5):
    """[M,B,T,H,d] -> [M*B, H, T, d] view of the same storage, or None where its strides allow none."""
    M, B, T, H, d = X5.shape
    try:
        return X5.permute(0, 1, 3, 2, 4).view(M * B, H, T, d)
    except RuntimeError:
        return None


def _bhtd_rows(X5):
    """[M*B, H, T, d] rows of X5 for the view entry points, which take one distinct row per
    (stream, token) with a token stride of at least d: a view of X5 where its strides give that,
    else a copy (an expanded tensor, e.g. the upstream gradient of out.sum(dim=2), has stride 0)."""
    M, B, T, H, d = X5.shape
    v = _bhtd(X5)
    if v is not None:
        z, h, t, _ = v.shape
        sz, sh, st, _ = v.stride()
        if st >= d and (h == 1 or sh > 0) and (z == 1 or sz > 0):
            return v
    return X5.permute(0, 1, 3, 2, 4).contiguous().view(M * B, H, T, d)


class RaceNonCausalViewFn(Function):
    """out [M,B,T,H,d] fp32 = RaceNonCausalFn of probsK / probsQ [M*B*H, T, S] (streams ordered
    (m, b, h)) and values Vhf [M,B,T,H,d]: values, output and their gradients stay in the
    [M,B,T,H,d] layout (race_nc_fwd_view / race_nc_bwd_view), where the reference permutes them to
    [N,T,d] and back (scaling/benchmark_time.py:116-128,164)."""

    @staticmethod
    def forward(ctx, probsK, probsQ, Vhf, eps):
        _lib.require_device(probsK, probsQ, Vhf)
        M, B, T, H, D = Vhf.shape
        N, S = M * B * H, probsK.shape[-1]
        if probsK.shape != (N, T, S) or probsQ.shape != probsK.shape:
            raise ValueError(f"probsK/probsQ must be [{N},{T},S], got {tuple(probsK.shape)}, {tuple(probsQ.shape)}")
        pK, pQ = probsK.contiguous().float(), probsQ.contiguous().float()
        Vv = _bhtd_rows(Vhf.float())
        out = torch.empty(M, B, T, H, D, dtype=torch.float32, device=Vv.device)
        lib = _lib.lib()
        state = state_buffer(lib.race_op_state_bytes(N, T, S, D, 0), Vv.device, "race_op_state_bytes")
        ws = _lib.workspace(lib.race_nc_op_workspace_bytes(N, T, S, D, 0, 0), Vv.device)
        vv, Vv = _lib.view4(Vv)
        ov, _ = _lib.view4(_bhtd(out))
        _lib.check(lib.race_nc_fwd_view(_lib.ptr(pK), _lib.ptr(pQ), vv, ov, M * B, H, T, S, D, float(eps), 0,
                                        _lib.ptr(ws), ws.numel(), *state_arg(state), _lib.stream_of(Vv)),
                   "race_nc_fwd_view")
        ctx.save_for_backward(pK, pQ, Vv, state)
        ctx.shape = (M, B, T, H, D)
        ctx.v_dtype = Vhf.dtype
        ctx.eps = float(eps)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        pK, pQ, Vv, state = ctx.saved_tensors
        M, B, T, H, D = ctx.shape
        N, S = pK.shape[0], pK.shape[2]
        gv_in = _bhtd_rows(grad_out.float())
        gpK, gpQ = torch.empty_like(pK), torch.empty_like(pQ)
        gV = torch.empty(M, B, T, H, D, dtype=torch.float32, device=pK.device)
        lib = _lib.lib()
        ws = _lib.workspace(lib.race_nc_op_workspace_bytes(N, T, S, D, 0, 1), pK.device)
        vv, _ = _lib.view4(Vv)
        gov, gv_in = _lib.view4(gv_in)
        gvv, _ = _lib.view4(_bhtd(gV))
        _lib.check(lib.race_nc_bwd_view(_lib.ptr(pK), _lib.ptr(pQ), vv, gov, _lib.ptr(gpK), _lib.ptr(gpQ), gvv, M * B,
                                        H, T, S, D, ctx.eps, 0, _lib.ptr(ws), ws.numel(), *state_arg(state),
                                        _lib.stream_of(pK)), "race_nc_bwd_view")
        return gpK, gpQ, gV.to(ctx.v_dtype), None


class SoftHashTempFn(Function):
    """Soft-hash probabilities [Mp*B*H, T, L*2^K] of X [B,H,T,D] with a learnable scale held in
    device memory (a 0-d fp32 tensor, as the reference's exp(logit_temp).clamp(1e-2, 10),
    scaling/benchmark_time.py:104,111): the kernels read it there, and the backward returns
    d loss / d X and d loss / d scale, reduced on the device. Nothing is read back to the host,
    so a forward+backward runs asynchronously and can be captured in a HIP graph."""

    @staticmethod
    def forward(ctx, X, planes_T, L, Kbits, M, unshared, scale):
        _lib.require_device(X, planes_T)
        B, H, T, D = X.shape
        if not torch.is_tensor(scale):
            scale = torch.tensor(float(scale), device=X.device)
        _lib.require_device(scale)
        sc = scale.detach().to(torch.float32).reshape(1).contiguous()
        planes = planes_T.detach().float().contiguous()
        xv, Xc = _lib.view4(X)
        Mp = M if unshared else 1
        probs = torch.empty(Mp * B * H, T, L << Kbits, dtype=torch.float32, device=X.device)
        sh = _hash_shape(X, L, Kbits, M, unshared, 1.0)  # the scale comes from sc
        _lib.check(_lib.lib().race_soft_hash_fwd_dscale(sh, xv, _lib.dtype_code(X.dtype), _lib.ptr(planes),
                                                        _lib.ptr(sc), _lib.ptr(probs), _lib.stream_of(X)),
                   "race_soft_hash_fwd_dscale")
        ctx.save_for_backward(Xc, planes, sc)
        ctx.cfg = (L, Kbits, M, unshared)
        ctx.scale_shape = scale.shape
        return probs

    @staticmethod
    def backward(ctx, gprobs):
        Xc, planes, sc = ctx.saved_tensors
        L, Kbits, M, unshared = ctx.cfg
        B, H, T, D = Xc.shape
        Mp = M if unshared else 1
        g = gprobs.float().contiguous().view(Mp, B * H, T, -1)
        # in X's own layout (a strided view of the caller's tensor): autograd hands it to the leaf
        # without a layout copy
        dX = torch.empty_like(Xc)
        xv, _ = _lib.view4(Xc)
        dv, _ = _lib.view4(dX)
        sh = _hash_shape(Xc, L, Kbits, Mp, unshared, 1.0)
        lib = _lib.lib()
        part = torch.empty(lib.race_soft_hash_bwd_partials(sh), dtype=torch.float32, device=Xc.device)
        dscale = torch.empty(1, dtype=torch.float32, device=Xc.device)
        _lib.check(lib.race_soft_hash_bwd_dscale(sh, xv, _lib.dtype_code(Xc.dtype), _lib.ptr(planes), _lib.ptr(sc),
                                                 _lib.ptr(g), dv, _lib.ptr(part), _lib.ptr(dscale),
                                                 _lib.stream_of(Xc)), "race_soft_hash_bwd_dscale")
        return dX, None, None, None, None, None, dscale.view(ctx.scale_shape)


class BatchedACE(nn.Module):
    """Non-causal BatchedACE (scaling/benchmark_time.py:77-166): Khf, Vhf, Qhf
    [M,B,T,H,d_k] -> [M,B,T,H,d_k], planes from the global RNG as the reference,
    learnable temperature logit_temp (scale = exp(logit_temp).clamp(1e-2, 10))."""

    def __init__(self, d_k, K, L, M, device="cpu", share_planes: bool = False):
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
        self.logit_temp = nn.Parameter(torch.log(torch.tensor(1.0, device=device)))

    def forward(self, Khf, Vhf, Qhf, eps: float = 1e-6):
        M, B, T, H, dk = Khf.shape
        if M != self.M or dk != self.d_k:
            raise ValueError(f"expected [M={self.M},B,T,H,{self.d_k}] inputs, got {tuple(Khf.shape)}")
        scale = self.logit_temp.exp().clamp(1e-2, 10.0)  # stays on the device (no host read)
        # streams ordered (M, B, H) as benchmark_time.py:121-131; one row of planes per m
        def bhtd(X):  # [M,B,T,H,dk] -> [M*B, H, T, dk] view
            return X.permute(0, 1, 3, 2, 4).reshape(M * B, H, T, dk)

        if self.share_planes:
            pK = SoftHashTempFn.apply(bhtd(Khf), self.planes_T, self.L, self.K, 1, False, scale)
            pQ = SoftHashTempFn.apply(bhtd(Qhf), self.planes_T, self.L, self.K, 1, False, scale)
        else:
            # per-ensemble planes [M, dk, L*K]: member m hashes its own B*H rows
            Kx = Khf.permute(0, 1, 3, 2, 4).reshape(M, B * H, T, dk)
            Qx = Qhf.permute(0, 1, 3, 2, 4).reshape(M, B * H, T, dk)
            pK = torch.cat([SoftHashTempFn.apply(Kx[m:m + 1], self.planes_T[m], self.L, self.K, 1, False, scale)
                            for m in range(M)], 0)
            pQ = torch.cat([SoftHashTempFn.apply(Qx[m:m + 1], self.planes_T[m], self.L, self.K, 1, False, scale)
                            for m in range(M)], 0)
        # values, output and gradients in the [M,B,T,H,dk] layout: no permute copies
        return RaceNonCausalViewFn.apply(pK, pQ, Vhf, eps)


def race_attention(Q, K, V, ace_module: BatchedACE, eps=1e-6):
    """[B,H,T,D] wrapper of BatchedACE (scaling/benchmark_time.py:168-176): pack to
    [M,B,T,H,D], run, average over M, return [B,H,T,D]."""
    M = ace_module.M

    def pack(Z):
        return Z.permute(0, 2, 1, 3).unsqueeze(0).expand(M, -1, -1, -1, -1)

    out = ace_module(pack(K), pack(V), pack(Q), eps)
    return out.mean(dim=0).permute(0, 2, 1, 3)
