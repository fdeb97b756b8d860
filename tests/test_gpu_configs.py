"""BASELINE.json configurations on the GPU.

cfg1 (the reference's CPU plumbing case, fp32) is checked whole against the fp64 oracle,
outputs and gradients, at both the reference's scale sqrt(D) and the literal temperature 1.0.
cfg2 and cfg3 are run at their full size (T = 65536 and T = 2^20); their outputs are checked
through causality, a size-independent property: the first T0 outputs of the full run depend
only on the first T0 tokens, so they must match the oracle evaluated on that prefix. The
backward at full size is checked for finiteness and bitwise determinism; its values are
pinned at smaller T by tests/test_gpu_fused.py.
"""
import math

import pytest
import torch

from race_ref import bf16_planes, check, oracle_layer

pytestmark = pytest.mark.gpu

EPS = 1e-6


@pytest.mark.parametrize("scale", [None, 1.0])
def test_cfg1_fp32_layer(dev, scale):
    """B=2, H=8, T=2048, D=64, L=8, K=4, fp32, q/k/v ~ N(0,1), upstream grad ~ N(0,1)."""
    from race_attention_amd import build_planes_protos
    from race_attention_amd.race_common import soft_hash_probs
    from race_attention_amd.race_causal_cuda import RaceCausalFn
    B, H, T, D, L, K = 2, 8, 2048, 64, 8, 4
    s = math.sqrt(D) if scale is None else scale
    g = torch.Generator().manual_seed(1)
    Q, Kt, V, go = (torch.randn(B, H, T, D, generator=g) for _ in range(4))
    planes_T, protos_T = build_planes_protos(D, K, L, 1, device=dev, seed=0)
    q, k, v = (x.to(dev).requires_grad_(True) for x in (Q, Kt, V))
    pK, pQ, V2, N = soft_hash_probs(q, k, v, planes_T, protos_T, L, K, 1, True, scale=s)
    out = RaceCausalFn.apply(pK, pQ, V2, EPS).view(B, H, T, D)
    out.backward(go.to(dev))
    ref, dq, dk, dv = oracle_layer(Q, Kt, V, planes_T.cpu(), L, K, s, EPS, go)
    check("cfg1 out", out, ref, 1e-4)
    check("cfg1 dq", q.grad, dq, 1e-4 if scale is None else 3e-3)
    check("cfg1 dk", k.grad, dk, 1e-4 if scale is None else 3e-3)
    check("cfg1 dv", v.grad, dv, 1e-4)


def _full_size(dev, B, Hq, Hkv, T, D, L, K, std, T0, seed):
    from race_attention_amd import build_planes_protos, race_causal_attention
    print(f"full-size B={B} H={Hq}/{Hkv} T={T} D={D} L={L} K={K}", flush=True)
    planes_T, _ = build_planes_protos(D, K, L, 1, device=dev, seed=0)
    g = torch.Generator(device=dev).manual_seed(seed)
    q = (torch.randn(B, Hq, T, D, generator=g, device=dev) * std).to(torch.bfloat16).requires_grad_(True)
    k = (torch.randn(B, Hkv, T, D, generator=g, device=dev) * std).to(torch.bfloat16).requires_grad_(True)
    v = (torch.randn(B, Hkv, T, D, generator=g, device=dev) * std).to(torch.bfloat16).requires_grad_(True)
    go = torch.randn(B, Hq, T, D, generator=g, device=dev).to(torch.bfloat16)
    out = race_causal_attention(q, k, v, planes_T, L, K, eps=EPS)
    out.backward(go)
    grads = [x.grad.clone() for x in (q, k, v)]
    ref = oracle_layer(q[..., :T0, :].detach(), k[..., :T0, :].detach(), v[..., :T0, :].detach(),
                       bf16_planes(planes_T).cpu(), L, K, math.sqrt(D), EPS)
    check(f"prefix of the full-size output (T0={T0})", out[..., :T0, :], ref, 2e-2)
    for x in grads:
        assert torch.isfinite(x.float()).all()
    # bitwise determinism of the full-size backward
    for x in (q, k, v):
        x.grad = None
    race_causal_attention(q, k, v, planes_T, L, K, eps=EPS).backward(go)
    for a, x in zip(grads, (q, k, v)):
        assert torch.equal(a, x.grad), "full-size backward is not deterministic"


def test_cfg2_full_size(dev):
    """B=4, H=16, T=65536, D=64, L=16, K=4 (S=256: two bucket tiles), bf16 ~ N(0,1)."""
    _full_size(dev, 4, 16, 16, 65536, 64, 16, 4, 1.0, T0=1024, seed=2)


def test_cfg3_full_size(dev):
    """B=1, H=4, T=2^20, D=64, L=8, K=4, bf16 ~ N(0, 1/sqrt(D))."""
    _full_size(dev, 1, 4, 4, 1 << 20, 64, 8, 4, 1.0 / math.sqrt(64), T0=2048, seed=1)
