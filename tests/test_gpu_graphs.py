"""HIP graph capture of the hot path (serving loops replay a captured decode step).

The library allocates nothing, issues no memset and launches on the caller's current stream, so
its kernels can be captured. Each test replays a captured graph several times, with the program's
own eager work and synchronisations between the replays, and checks every replay bitwise against
the same computation run eagerly.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def test_decode_step_graph_replays_equal_eager(dev):
    from race_attention_amd import RaceDecodeState, build_planes_protos
    B, Hq, Hkv, D, L, Kb = 4, 8, 2, 64, 8, 4
    planes_T, _ = build_planes_protos(D, Kb, L, 1, device=dev, seed=5)
    g = torch.Generator(device=dev).manual_seed(11)

    def draw():
        return (torch.randn(B, Hq, D, generator=g, device=dev).bfloat16(),
                torch.randn(B, Hkv, D, generator=g, device=dev).bfloat16(),
                torch.randn(B, Hkv, D, generator=g, device=dev).bfloat16())

    # code objects loaded and library initialised before capture
    warm = RaceDecodeState(B, Hq, Hkv, D, L, Kb, planes_T, device=dev)
    warm.step(*draw())
    torch.cuda.synchronize()

    eager = RaceDecodeState(B, Hq, Hkv, D, L, Kb, planes_T, device=dev)
    graphed = RaceDecodeState(B, Hq, Hkv, D, L, Kb, planes_T, device=dev)
    q_s, k_s, v_s = (torch.zeros_like(x) for x in draw())
    out_s = torch.empty_like(q_s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        graphed.step(q_s, k_s, v_s, out=out_s)
    torch.cuda.synchronize()
    # capture records the step without running it: the captured state is still empty
    assert not graphed.A.any() and not graphed.Bs.any()

    for i in range(6):
        q, k, v = draw()
        q_s.copy_(q)
        k_s.copy_(k)
        v_s.copy_(v)
        graph.replay()
        o = eager.step(q, k, v)
        torch.cuda.synchronize()
        assert torch.equal(out_s, o), f"replay {i}: output differs from the eager step"
        assert torch.equal(graphed.A, eager.A), f"replay {i}: state A differs"
        assert torch.equal(graphed.Bs, eager.Bs), f"replay {i}: state Bs differs"


def test_layer_forward_graph_replays_equal_eager(dev):
    from race_attention_amd import build_planes_protos, race_causal_attention
    B, H, T, D, L, Kb = 1, 2, 3000, 64, 8, 4
    planes_T, _ = build_planes_protos(D, Kb, L, 1, device=dev, seed=6)
    g = torch.Generator(device=dev).manual_seed(12)

    def draw():
        return [(torch.randn(B, H, T, D, generator=g, device=dev) * 0.125).bfloat16() for _ in range(3)]

    race_causal_attention(*draw(), planes_T, L, Kb)
    torch.cuda.synchronize()
    static = [torch.zeros(B, H, T, D, device=dev, dtype=torch.bfloat16) for _ in range(3)]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_s = race_causal_attention(*static, planes_T, L, Kb)
    torch.cuda.synchronize()

    for i in range(4):
        x = draw()
        for s, t in zip(static, x):
            s.copy_(t)
        graph.replay()
        ref = race_causal_attention(*x, planes_T, L, Kb)
        torch.cuda.synchronize()
        assert torch.equal(out_s, ref), f"replay {i}: output differs from the eager forward"


def test_layer_forward_backward_graph_replays_equal_eager(dev):
    from race_attention_amd import build_planes_protos, race_causal_attention
    B, H, T, D, L, Kb = 1, 2, 2500, 64, 8, 4
    planes_T, _ = build_planes_protos(D, Kb, L, 1, device=dev, seed=7)
    g = torch.Generator(device=dev).manual_seed(13)

    def draw():
        return [(torch.randn(B, H, T, D, generator=g, device=dev) * 0.125).bfloat16() for _ in range(4)]

    def step(q, k, v, go):
        out = race_causal_attention(q, k, v, planes_T, L, Kb)
        out.backward(go)
        return out

    leaves = [torch.zeros(B, H, T, D, device=dev, dtype=torch.bfloat16, requires_grad=True) for _ in range(3)]
    go_s = torch.zeros(B, H, T, D, device=dev, dtype=torch.bfloat16)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on a side stream, as torch's whole-step capture expects
        for _ in range(2):
            step(*leaves, go_s)
            for t in leaves:
                t.grad = None
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_s = step(*leaves, go_s)
    torch.cuda.synchronize()

    for i in range(3):
        x = draw()
        with torch.no_grad():
            for s, t in zip(leaves + [go_s], x):
                s.copy_(t)
        graph.replay()
        ref_leaves = [t.clone().requires_grad_(True) for t in x[:3]]
        ref = step(*ref_leaves, x[3])
        torch.cuda.synchronize()
        assert torch.equal(out_s, ref), f"replay {i}: output differs"
        for name, a, b in zip("qkv", leaves, ref_leaves):
            assert torch.equal(a.grad, b.grad), f"replay {i}: d{name} differs"
