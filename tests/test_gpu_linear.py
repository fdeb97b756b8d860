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


def test_causal_linear_destinations(dev):
    """Outputs written in place when contiguous fp32, through a temporary otherwise: a strided
    destination, and a destination that is the value tensor itself (the kernels read their
    inputs in several passes, so an aliased output must not be written directly)."""
    from race_attention_amd.linear_attention import causal_dot_backward, causal_dot_product
    N, H, L, E = 1, 2, 700, 32
    g = torch.Generator().manual_seed(3)
    Q, K, V, G = (torch.randn(N, H, L, E, generator=g) for _ in range(4))
    q1, k1, v1 = (x.double().requires_grad_(True) for x in (Q, K, V))
    ref = orc.causal_linear_ref(q1, k1, v1)
    ref.backward(G.double())
    Qd, Kd, Vd, Gd = (x.to(dev) for x in (Q, K, V, G))
    strided = torch.zeros(N, L, H, E, device=dev).transpose(1, 2)  # [N,H,L,E] view, not contiguous
    causal_dot_product(Qd, Kd, Vd, strided)
    check("strided product", strided, ref, 1e-3)
    Va = Vd.clone()
    causal_dot_product(Qd, Kd, Va, Va)  # product aliases the values
    check("aliased product", Va, ref, 1e-3)
    gq, gk = torch.empty_like(Qd), torch.zeros(N, L, H, E, device=dev).transpose(1, 2)
    Ga = Gd.clone()
    causal_dot_backward(Qd, Kd, Vd, Ga, gq, gk, Ga)  # grad_values aliases grad_out
    check("gQ", gq, q1.grad, 2e-3)
    check("gK (strided)", gk, k1.grad, 2e-3)
    check("gV (aliased)", Ga, v1.grad, 2e-3)


def test_causal_linear_backward_from_kept_state(dev):
    """causal_dot_backward reading the forward's kept block states (CausalLinearFn's path) is
    bitwise the one that recomputes them, also when called twice on the same state."""
    from race_attention_amd.linear_attention import causal_dot_backward, causal_dot_product, linear_state
    g = torch.Generator(device=dev).manual_seed(4)
    Q, K, V, G = (torch.randn(2, 2, 3000, 32, generator=g, device=dev) for _ in range(4))
    st = linear_state(Q, V)
    a, b = torch.empty_like(V), torch.empty_like(V)
    causal_dot_product(Q, K, V, a, state=st)
    causal_dot_product(Q, K, V, b)
    assert torch.equal(a, b)
    ref = [torch.empty_like(x) for x in (Q, K, V)]
    causal_dot_backward(Q, K, V, G, *ref)
    for rep in range(2):
        got = [torch.empty_like(x) for x in (Q, K, V)]
        causal_dot_backward(Q, K, V, G, *got, state=st)
        for name, x, y in zip(("gQ", "gK", "gV"), got, ref):
            assert torch.equal(x, y), f"call {rep}: {name} from the kept state differs"
