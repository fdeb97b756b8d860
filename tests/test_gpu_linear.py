"""Causal linear attention (kernels/cpu/linear_pref.cpp:87-213) on the GPU, against the
fp64 oracle with the reference test's sweeps and tolerances (kernels/cpu/
test_cpu_kernels.py:100-139: forward 1e-3, gradients 2e-3), extended to longer L."""
import pytest
import torch

from oracle import race_oracle as orc
from race_ref import check

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,H,L,E,M", [(1, 1, 1, 4, 4), (2, 2, 16, 8, 8), (2, 4, 256, 32, 32),
                                       (1, 2, 2048, 64, 64), (1, 2, 1024, 64, 64), (1, 1, 5000, 128, 96),
                                       (2, 1, 333, 300, 40)])
def test_causal_linear(dev, N, H, L, E, M):
    from race_attention_amd.linear_attention import CausalLinearFn, causal_dot_product
    print(f"linear N={N} H={H} L={L} E={E} M={M}", flush=True)
    g = torch.Generator().manual_seed(L + E)
    Q, K, V = torch.randn(N, H, L, E, generator=g), torch.randn(N, H, L, E, generator=g), torch.randn(N, H, L, M, generator=g)
    Wl = torch.randn(N, H, L, M, generator=g)
    q1, k1, v1 = (x.double().requires_grad_(True) for x in (Q, K, V))
    ref = orc.causal_linear_ref(q1, k1, v1)
    (ref * Wl.double()).sum().backward()
    out = torch.zeros(N, H, L, M, device=dev)
    causal_dot_product(Q.to(dev), K.to(dev), V.to(dev), out)
    check("linear fwd", out, ref, 1e-3)
    q2, k2, v2 = (x.to(dev).requires_grad_(True) for x in (Q, K, V))
    (CausalLinearFn.apply(q2, k2, v2) * Wl.to(dev)).sum().backward()
    check("linear gQ", q2.grad, q1.grad, 2e-3)
    check("linear gK", k2.grad, k1.grad, 2e-3)
    check("linear gV", v2.grad, v1.grad, 2e-3)
