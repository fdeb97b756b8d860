"""Non-causal RACE (BatchedACE, scaling/benchmark_time.py:77-176) on the GPU against the
fp64 oracle: the probability-level op (RaceNonCausalFn over race_nc_op_fwd/bwd) and the
module with its learnable temperature (soft-hash backward with d loss / d scale).
fp32 throughout: tolerance 1e-4 (max-normalised, scaling/test_kernels.py:30-31)."""
import pytest
import torch

from oracle import race_oracle as orc
from race_ref import check

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _probs(N, T, S, D, seed):
    g = torch.Generator().manual_seed(seed)
    pk = torch.softmax(torch.randn(N, T, S, generator=g) * 2, -1)
    pq = torch.softmax(torch.randn(N, T, S, generator=g) * 2, -1)
    v = torch.randn(N, T, D, generator=g)
    go = torch.randn(N, T, D, generator=g)
    return pk, pq, v, go


# S <= 32 (any D), S <= 64 (D <= 128) and S <= 128 (D <= 64) take the matrix-core kernels (ragged S
# and D: 30 x 100, 1 x 20, 32 x 64, 40 x 120, 100 x 50);
# the last two: enough token tiles that each workgroup walks several (ragged last tile), with every
# bucket in one chunk (S = 24) and over several chunks (S = 64)
@pytest.mark.parametrize("N,T,S,D", [(1, 1, 8, 16), (2, 7, 24, 64), (3, 300, 128, 64), (1, 4096, 256, 128),
                                     (2, 1000, 64, 100), (2, 1000, 30, 100), (3, 517, 32, 64), (1, 77, 1, 20),
                                     (2, 555, 40, 120), (2, 777, 100, 50),
                                     (1, 513, 300, 256), (2, 333, 24, 256), (4, 2000, 16, 32),
                                     (4, 70001, 24, 128), (4, 66017, 64, 32)])
def test_noncausal_op(dev, N, T, S, D):
    from race_attention_amd.noncausal import RaceNonCausalFn
    print(f"nc op N={N} T={T} S={S} D={D}", flush=True)
    pk, pq, v, go = _probs(N, T, S, D, seed=T + S + D)
    eps = 1e-6
    pkr, pqr, vr = (x.double().requires_grad_(True) for x in (pk, pq, v))
    ref = orc.race_noncausal_ref(pkr, pqr, vr, eps)
    ref.backward(go.double())
    pkx, pqx, vx = (x.to(dev).requires_grad_(True) for x in (pk, pq, v))
    out = RaceNonCausalFn.apply(pkx, pqx, vx, eps)
    out.backward(go.to(dev))
    check("out", out, ref, TOL)
    check("gpK", pkx.grad, pkr.grad, TOL)
    check("gpQ", pqx.grad, pqr.grad, TOL)
    check("gV", vx.grad, vr.grad, TOL)


@pytest.mark.parametrize("S,D,pad", [(24, 128, 0), (30, 100, 1), (64, 64, 3), (100, 120, 1), (256, 64, 0)])
def test_noncausal_view_layouts(dev, S, D, pad):
    """race_nc_fwd_view / race_nc_bwd_view (RaceNonCausalViewFn): values and upstream gradient as
    [M,B,T,H,D] slices of wider rows (odd pad: token and head strides not multiples of 4, rows
    moved element-wise), output and gV written in [M,B,T,H,D], against the fp64 oracle on the
    same streams in [N,T,D]. The first three shapes run the matrix-core kernels (S <= 32, and
    S = 64 at D <= 128 padded to 64 buckets); S = 100 at D = 120 and S = 256 run the FMA readout
    and backward, whose rows are addressed per head through the same strided views."""
    from race_attention_amd.noncausal import RaceNonCausalViewFn
    M, B, T, H = 2, 2, 777, 3
    N = M * B * H
    print(f"nc view S={S} D={D} pad={pad}", flush=True)
    g = torch.Generator().manual_seed(S + D + pad)
    pk = torch.softmax(torch.randn(N, T, S, generator=g) * 2, -1)
    pq = torch.softmax(torch.randn(N, T, S, generator=g) * 2, -1)
    vfull = torch.randn(M, B, T, H, D + pad, generator=g)
    gfull = torch.randn(M, B, T, H, D + pad, generator=g)
    v5, go5 = vfull[..., :D], gfull[..., :D]
    eps = 1e-6

    def flat(x5):
        return x5.permute(0, 1, 3, 2, 4).reshape(N, T, D)

    pkr, pqr, vr = pk.double().requires_grad_(True), pq.double().requires_grad_(True), \
        flat(v5).double().requires_grad_(True)
    ref = orc.race_noncausal_ref(pkr, pqr, vr, eps)
    ref.backward(flat(go5).double())
    pkx, pqx = pk.to(dev).requires_grad_(True), pq.to(dev).requires_grad_(True)
    vx = vfull.to(dev)[..., :D].detach().requires_grad_(True)
    out = RaceNonCausalViewFn.apply(pkx, pqx, vx, eps)
    assert out.shape == (M, B, T, H, D)
    out.backward(gfull.to(dev)[..., :D])
    check("out", flat(out), ref, TOL)
    check("gpK", pkx.grad, pkr.grad, TOL)
    check("gpQ", pqx.grad, pqr.grad, TOL)
    check("gV", flat(vx.grad), vr.grad, TOL)


def test_noncausal_unaligned_buffers(dev):
    """Contiguous probabilities, values and upstream gradient that start 4 bytes past a 16-byte
    boundary: the matrix-core kernels take their element-wise paths (no 16-byte runs) and agree with
    the fp64 oracle as the aligned case does."""
    from race_attention_amd.noncausal import RaceNonCausalFn
    N, T, S, D = 2, 1000, 24, 128
    pk, pq, v, go = _probs(N, T, S, D, seed=5)

    def odd(x):  # same values, data pointer 4 bytes past 16-byte alignment
        buf = torch.empty(x.numel() + 1, dtype=x.dtype, device=dev)
        y = buf[1:].view(x.shape)
        y.copy_(x.to(dev))
        assert y.is_contiguous() and y.data_ptr() % 16 == 4
        return y

    eps = 1e-6
    pkr, pqr, vr = (x.double().requires_grad_(True) for x in (pk, pq, v))
    ref = orc.race_noncausal_ref(pkr, pqr, vr, eps)
    ref.backward(go.double())
    pkx, pqx, vx = (odd(x).requires_grad_(True) for x in (pk, pq, v))
    out = RaceNonCausalFn.apply(pkx, pqx, vx, eps)
    out.backward(odd(go))
    check("out", out, ref, TOL)
    check("gpK", pkx.grad, pkr.grad, TOL)
    check("gpQ", pqx.grad, pqr.grad, TOL)
    check("gV", vx.grad, vr.grad, TOL)


@pytest.mark.parametrize("S", [40, 24])
def test_noncausal_unaligned_gradient_outputs(dev, S):
    """race_nc_op_bwd through the C ABI with gpQ / gpK 4 bytes past 16-byte alignment (S = 40: the
    64-bucket matrix-core backward; S = 24: the 32-bucket one with its probability-tile path): the
    gradients are stored element-wise and equal the call with aligned outputs bitwise."""
    from race_attention_amd import _lib
    N, T, D, eps = 2, 1500, 64, 1e-6
    pk, pq, v, go = (x.to(dev) for x in _probs(N, T, S, D, seed=S + 77))
    lib = _lib.lib()
    ws = _lib.workspace(lib.race_nc_op_workspace_bytes(N, T, S, D, 0, 1), dev)

    def run(gpK, gpQ):
        gV = torch.empty(N, T, D, device=dev)
        _lib.check(lib.race_nc_op_bwd(_lib.ptr(pk), _lib.ptr(pq), _lib.ptr(v), _lib.ptr(go), _lib.ptr(gpK),
                                      _lib.ptr(gpQ), _lib.ptr(gV), N, T, S, D, eps, 0, _lib.ptr(ws), ws.numel(),
                                      _lib.stream_of(pk)), "race_nc_op_bwd")
        return gV

    def odd():
        buf = torch.full((N * T * S + 1,), float("nan"), device=dev)
        y = buf[1:].view(N, T, S)
        assert y.data_ptr() % 16 == 4
        return y

    a_k, a_q = torch.empty(N, T, S, device=dev), torch.empty(N, T, S, device=dev)
    gv_a = run(a_k, a_q)
    o_k, o_q = odd(), odd()
    gv_o = run(o_k, o_q)
    torch.cuda.synchronize()
    assert torch.equal(o_k, a_k) and torch.equal(o_q, a_q) and torch.equal(gv_o, gv_a)


@pytest.mark.parametrize("S", [64, 24, 160])
def test_noncausal_block_invariance(dev, S):
    """The totals over any block split agree to fp32 rounding (S = 24 and S = 64 at D = 64: one
    bucket tile of the totals kernel, with the matrix-core readout; S = 160: three 64-bucket tiles,
    with the FMA readout)."""
    from race_attention_amd.noncausal import race_nc_fwd
    pk, pq, v, _ = _probs(2, 3000, S, 64, seed=9)
    a = race_nc_fwd(pk.to(dev), pq.to(dev), v.to(dev), 1e-6, 0)
    for blk in (16, 256, 3000):
        b = race_nc_fwd(pk.to(dev), pq.to(dev), v.to(dev), 1e-6, blk)
        check(f"block {blk}", b, a.double(), 1e-6)


@pytest.mark.parametrize("share", [True, False])
@pytest.mark.parametrize("M", [1, 2])
def test_batched_ace_noncausal_module(dev, share, M):
    from race_attention_amd.noncausal import BatchedACE, race_attention
    torch.manual_seed(0)
    B, T, H, dk, L, K = 2, 200, 3, 64, 4, 3
    ace = BatchedACE(dk, K, L, M, device=dev, share_planes=share)
    with torch.no_grad():
        ace.logit_temp.fill_(0.4)
    g = torch.Generator().manual_seed(1)
    Kh, Vh, Qh = (torch.randn(M, B, T, H, dk, generator=g) for _ in range(3))
    go = torch.randn(M, B, T, H, dk, generator=g)
    lt = torch.tensor(0.4, dtype=torch.float64, requires_grad=True)
    refs = [x.double().requires_grad_(True) for x in (Kh, Vh, Qh)]
    ref = orc.batched_ace_nc_ref(*refs, ace.planes_T.cpu(), ace.protos_T.cpu(), L, K, share, lt)
    ref.backward(go.double())
    xs = [x.to(dev).requires_grad_(True) for x in (Kh, Vh, Qh)]
    out = ace(*xs)
    out.backward(go.to(dev))
    check("out", out, ref, TOL)
    for name, a, r in zip(("dK", "dV", "dQ"), xs, refs):
        check(name, a.grad, r.grad, TOL)
    check("dlogit_temp", ace.logit_temp.grad.reshape(1), lt.grad.reshape(1), TOL)
    # [B,H,T,D] wrapper: mean over the M copies of the same inputs
    Q4, K4, V4 = (torch.randn(B, H, T, dk, generator=g).to(dev) for _ in range(3))
    with torch.no_grad():
        o4 = race_attention(Q4, K4, V4, ace)
        pack = lambda Z: Z.permute(0, 2, 1, 3).unsqueeze(0).expand(M, -1, -1, -1, -1).double().cpu()
        r4 = orc.batched_ace_nc_ref(pack(K4), pack(V4), pack(Q4), ace.planes_T.cpu(), ace.protos_T.cpu(), L, K,
                                    share, lt.detach()).mean(0).permute(0, 2, 1, 3)
    check("race_attention", o4, r4, TOL)


def test_batched_ace_broadcast_upstream_gradient(dev):
    """A loss over out.sum(dim=2) hands the backward an upstream gradient expanded along T
    (token stride 0): the module copies it to distinct rows and the gradients match fp64."""
    from race_attention_amd.noncausal import BatchedACE
    torch.manual_seed(0)
    M, B, T, H, dk, L, K = 2, 2, 300, 3, 64, 4, 3
    ace = BatchedACE(dk, K, L, M, device=dev, share_planes=True)
    g = torch.Generator().manual_seed(3)
    Kh, Vh, Qh = (torch.randn(M, B, T, H, dk, generator=g) for _ in range(3))
    w = torch.randn(M, B, H, dk, generator=g)
    lt = torch.tensor(0.0, dtype=torch.float64, requires_grad=True)
    refs = [x.double().requires_grad_(True) for x in (Kh, Vh, Qh)]
    ref = orc.batched_ace_nc_ref(*refs, ace.planes_T.cpu(), ace.protos_T.cpu(), L, K, True, lt)
    (ref.sum(dim=2) * w.double()).sum().backward()
    xs = [x.to(dev).requires_grad_(True) for x in (Kh, Vh, Qh)]
    out = ace(*xs)
    (out.sum(dim=2) * w.to(dev)).sum().backward()
    for name, a, r in zip(("dK", "dV", "dQ"), xs, refs):
        check(name, a.grad, r.grad, TOL)
    check("dlogit_temp", ace.logit_temp.grad.reshape(1), lt.grad.reshape(1), TOL)


def test_batched_ace_graph_replays_equal_eager(dev):
    """The temperature stays in device memory (no host read per call), so a BatchedACE
    forward+backward captures into a HIP graph: every replay's output and gradients, the
    temperature's included, equal the eager call bitwise."""
    from race_attention_amd.noncausal import BatchedACE
    torch.manual_seed(0)
    M, B, T, H, dk, L, K = 1, 2, 1000, 4, 64, 3, 3
    ace = BatchedACE(dk, K, L, M, device=dev, share_planes=True)
    with torch.no_grad():
        ace.logit_temp.fill_(0.3)
    g = torch.Generator(device=dev).manual_seed(21)

    def draw():
        return [torch.randn(M, B, T, H, dk, generator=g, device=dev) for _ in range(4)]

    def step(kh, vh, qh, go):
        out = ace(kh, vh, qh)
        out.backward(go)
        return out

    leaves = [torch.zeros(M, B, T, H, dk, device=dev, requires_grad=True) for _ in range(3)]
    go_s = torch.zeros(M, B, T, H, dk, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on a side stream, as torch's whole-step capture expects
        for _ in range(2):
            step(*leaves, go_s)
            for t in leaves:
                t.grad = None
            ace.logit_temp.grad = None
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_s = step(*leaves, go_s)
    torch.cuda.synchronize()
    gt_s = ace.logit_temp.grad
    for i in range(3):
        x = draw()
        with torch.no_grad():
            for s_, t in zip(leaves + [go_s], x):
                s_.copy_(t)
        graph.replay()
        got = [out_s.clone()] + [t.grad.clone() for t in leaves] + [gt_s.clone()]
        ace.logit_temp.grad = None
        ref_leaves = [t.clone().requires_grad_(True) for t in x[:3]]
        ref = step(*ref_leaves, x[3])
        torch.cuda.synchronize()
        exp = [ref] + [t.grad for t in ref_leaves] + [ace.logit_temp.grad]
        ace.logit_temp.grad = gt_s  # the graph's static gradient buffer
        for name, a, b in zip(("out", "dK", "dV", "dQ", "dlogit_temp"), got, exp):
            assert torch.equal(a, b), f"replay {i}: {name} differs from the eager call"


def test_soft_hash_temperature_grad_multi_tile(dev):
    """d loss / d scale summed from the per-workgroup partials when every workgroup walks several
    32-token tiles (2 per workgroup here, ragged last tile), against the fp64 softmax form."""
    from race_attention_amd import build_planes_protos
    from race_attention_amd.noncausal import SoftHashTempFn
    L, Kb, D, B, H, T = 2, 2, 64, 4, 8, 4141
    planes_T, protos_T = build_planes_protos(D, Kb, L, 1, device=dev, seed=6)
    g = torch.Generator().manual_seed(6)
    X = torch.randn(B, H, T, D, generator=g)
    gp = torch.randn(B * H, T, L << Kb, generator=g)
    xd = X.to(dev).requires_grad_(True)
    sd = torch.tensor(0.7, device=dev, requires_grad=True)
    p = SoftHashTempFn.apply(xd, planes_T, L, Kb, 1, False, sd)
    p.backward(gp.to(dev))
    X64 = X.double().requires_grad_(True)
    s64 = torch.tensor(0.7, dtype=torch.float64, requires_grad=True)
    ref, _, _, _ = orc.soft_hash_probs(X64.detach(), X64, X64.detach(), planes_T.cpu(), protos_T.cpu(), L, Kb,
                                       scale=s64)
    ref.backward(gp.double())
    check("probs", p, ref.detach(), 1e-5)
    check("dX", xd.grad, X64.grad, 1e-4)
    check("dscale", sd.grad.reshape(1), s64.grad.reshape(1), 1e-4)


def test_soft_hash_extreme_temperature(dev):
    """Temperature at BatchedACE's lower clamp (scale 0.01, scaling/benchmark_time.py:111):
    u = tanh(proj) / scale reaches +-100, where exp(-2u) overflows fp32 unless the corner
    sigmoid's argument is bounded. Probabilities, d/dX and d/dscale stay finite and match the
    fp64 softmax form (scaling/race_common.py:68-72)."""
    from race_attention_amd import build_planes_protos
    from race_attention_amd.noncausal import SoftHashTempFn
    L, Kb, D = 4, 3, 64
    planes_T, protos_T = build_planes_protos(D, Kb, L, 1, device=dev, seed=3)
    g = torch.Generator().manual_seed(5)
    X = torch.randn(1, 2, 300, D, generator=g) * 2
    gp = torch.randn(2, 300, L << Kb, generator=g)
    xd = X.to(dev).requires_grad_(True)
    sd = torch.tensor(0.01, device=dev, requires_grad=True)
    p = SoftHashTempFn.apply(xd, planes_T, L, Kb, 1, False, sd)
    p.backward(gp.to(dev))
    X64 = X.double().requires_grad_(True)
    s64 = torch.tensor(0.01, dtype=torch.float64, requires_grad=True)
    ref, _, _, _ = orc.soft_hash_probs(X64.detach(), X64, X64.detach(), planes_T.cpu(), protos_T.cpu(), L, Kb,
                                       scale=s64)  # first output: probabilities of the K argument
    ref.backward(gp.double())
    assert torch.isfinite(p).all() and torch.isfinite(xd.grad).all() and torch.isfinite(sd.grad).all()
    assert float(ref.detach().abs().max()) > 0.99  # saturated corners: the regime under test
    # At this temperature the reference formula itself, evaluated in fp32 (torch softmax form,
    # the reference's arithmetic), is ~1e-4 from fp64 (1 - tanh^2 near saturation, x 1/scale):
    # the bar is twice that fp32 floor, and never looser than it would be at 1e-4.
    X32 = X.clone().requires_grad_(True)
    s32 = torch.tensor(0.01, requires_grad=True)
    proj32 = (X32.reshape(-1, D) @ planes_T.cpu()).view(2, 300, L, Kb)
    r32 = torch.softmax((proj32.tanh() / s32) @ protos_T.cpu(), -1).reshape(2, 300, -1)
    r32.backward(gp)
    for name, got, g32, g64 in (("probs", p, r32.detach(), ref.detach()), ("dX", xd.grad, X32.grad, X64.grad),
                                ("dscale", sd.grad.reshape(1), s32.grad.reshape(1), s64.grad.reshape(1))):
        floor = orc.relerr(g32, g64)
        check(name, got, g64, max(TOL, 2.0 * floor))


def test_noncausal_backward_from_kept_totals(dev):
    """race_nc_bwd reading the forward's kept totals (RaceNonCausalFn's path) is bitwise the one
    that recomputes them; the state is only read, so a second backward on it is equal."""
    from race_attention_amd.noncausal import race_nc_bwd, race_nc_fwd
    from race_attention_amd.race_causal_cuda import op_state
    pk, pq, v, go = (x.to(dev) for x in _probs(2, 5000, 24, 64, seed=31))
    state = op_state(pk, v)
    assert torch.equal(race_nc_fwd(pk, pq, v, 1e-6, state=state), race_nc_fwd(pk, pq, v, 1e-6))
    ref = race_nc_bwd(pk, pq, v, go, 1e-6)
    for rep in range(2):
        got = race_nc_bwd(pk, pq, v, go, 1e-6, state=state)
        for name, a, b in zip(("gpK", "gpQ", "gV"), got, ref):
            assert torch.equal(a, b), f"call {rep}: {name} from the kept totals differs"
