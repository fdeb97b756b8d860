"""Pins the CPU oracle before anything is checked against it (runs without a GPU).

Each oracle function is checked against something independent of its own
formula: a second formula (softmax vs product of sigmoids), explicit loops,
closed-form known answers, finite differences (gradcheck), the C restatement of
the reference's CPU kernel, the reference's own compiled kernel (oracle/_ref,
when built) and golden vectors written by the reference (tests/golden).
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle_c, race_cpu_port
from oracle import race_oracle as orc

F64 = torch.float64
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "soft_hash_golden.npz")


def softmax_probs(N, T, L, R, gen):
    return torch.softmax(torch.randn(N, T, L, R, generator=gen, dtype=F64), -1).reshape(N, T, L * R)


# ----------------------------------------------------------------------------- a1
def test_corners_are_binary_counting():
    for Kb in (1, 2, 3, 4):
        _, protos = orc.build_planes_protos(8, Kb, 2)
        R = 1 << Kb
        for r in range(R):
            for k in range(Kb):
                bit = (r >> (Kb - 1 - k)) & 1
                assert protos[k, r].item() == (1.0 if bit else -1.0)


def test_planes_match_reference_golden():
    z = np.load(GOLDEN)
    for i in range(6):
        B, H, T, D, L, Kb, seed, _ = z[f"c{i}_meta"]
        planes_T, protos_T = orc.build_planes_protos(int(D), int(Kb), int(L), seed=int(seed))
        assert np.array_equal(planes_T.numpy(), z[f"c{i}_planes_T"])
        assert np.array_equal(protos_T.numpy(), z[f"c{i}_protos_T"])


def test_planes_unshared_layout():
    pl, _ = orc.build_planes_protos(16, 3, 4, M=3, share_planes=False, seed=5)
    g = torch.Generator().manual_seed(5)
    raw = torch.randn(3, 4, 3, 16, generator=g)
    assert pl.shape == (3, 16, 12)
    # column j = l*K + k of ensemble m is plane (m, l, k)
    assert torch.equal(pl[2, :, 1 * 3 + 2], raw[2, 1, 2])


# ----------------------------------------------------------------------------- a2
@pytest.mark.parametrize("L,Kb,scale", [(2, 2, None), (8, 4, None), (3, 3, 1.0), (16, 4, 1.0)])
def test_softhash_softmax_equals_sigmoid_product(L, Kb, scale):
    g = torch.Generator().manual_seed(L * 10 + Kb)
    B, H, T, D = 2, 2, 9, 32
    X = torch.randn(B, H, T, D, generator=g, dtype=F64) * 3
    planes_T, protos_T = orc.build_planes_protos(D, Kb, L, seed=3)
    p_soft = orc.soft_hash_probs(X, X, X, planes_T, protos_T, L, Kb, scale=scale)[0]
    p_sig = orc.soft_hash_sigmoid(X, planes_T, L, Kb, scale=scale)
    assert (p_soft - p_sig).abs().max().item() < 1e-14
    R = 1 << Kb
    sums = p_soft.view(B * H, T, L, R).sum(-1)
    assert (sums - 1).abs().max().item() < 1e-14


def test_softhash_zero_planes_uniform_and_k1():
    X = torch.randn(1, 1, 5, 8, generator=torch.Generator().manual_seed(71), dtype=F64)
    _, protos = orc.build_planes_protos(8, 3, 2)
    p = orc.soft_hash_probs(X, X, X, torch.zeros(8, 6), protos, 2, 3)[0]
    assert torch.all(p == 1.0 / 8)
    # K=1: logits (-u, +u) -> [sigmoid(-2u), sigmoid(2u)]
    planes_T, protos1 = orc.build_planes_protos(8, 1, 1, seed=1)
    p1 = orc.soft_hash_probs(X, X, X, planes_T, protos1, 1, 1)[0]
    u = torch.tanh(X.view(5, 8) @ planes_T.to(F64)) / math.sqrt(8)
    # the two-way softmax and the sigmoid agree to a few ulp of values <= 1
    assert torch.allclose(p1[0, :, 0], torch.sigmoid(-2 * u[:, 0]), atol=1e-14)
    assert torch.allclose(p1[0, :, 1], torch.sigmoid(2 * u[:, 0]), atol=1e-15)


def test_softhash_against_reference_golden():
    """fp32 golden: bit-level agreement to fp32 rounding; bf16 golden: the reference's
    own bf16 roundings stay within the bf16 parity tolerance of the fp64 oracle."""
    z = np.load(GOLDEN)
    for i in range(6):
        B, H, T, D, L, Kb, seed, is_bf16 = (int(x) for x in z[f"c{i}_meta"])
        Q, K, V = (torch.from_numpy(z[f"c{i}_{n}"]) for n in "QKV")
        planes_T = torch.from_numpy(z[f"c{i}_planes_T"])
        protos_T = torch.from_numpy(z[f"c{i}_protos_T"])
        if is_bf16:  # the reference casts the planes to the input dtype (race_common.py:54)
            planes_T = planes_T.to(torch.bfloat16).float()
        pK, pQ, _, _ = orc.soft_hash_probs(Q, K, V, planes_T, protos_T, L, Kb)
        tol = 2e-2 if is_bf16 else 1e-6
        assert orc.relerr(torch.from_numpy(z[f"c{i}_probsK"]), pK) < tol
        assert orc.relerr(torch.from_numpy(z[f"c{i}_probsQ"]), pQ) < tol


# ----------------------------------------------------------------------------- a3
def test_prefix_ref_equals_brute_force():
    g = torch.Generator().manual_seed(0)
    N, T, L, R, D = 2, 7, 3, 4, 5
    pk, pq = softmax_probs(N, T, L, R, g), softmax_probs(N, T, L, R, g)
    v = torch.randn(N, T, D, generator=g, dtype=F64)
    out, A, B = orc.race_prefix_ref(pk, pq, v, 1e-6)
    assert (out - orc.race_prefix_brute(pk, pq, v, 1e-6)).abs().max().item() < 1e-13
    assert torch.allclose(A, pk.sum(1)) and torch.allclose(B, torch.einsum("nts,ntd->nsd", pk, v))


def test_prefix_ref_zero_planes_known_answer():
    """planes = 0 -> p = 1/R everywhere -> out_t = L * sum_{tau<=t} v / (t+1+R*eps)."""
    L, Kb, eps = 4, 3, 1e-3
    R = 1 << Kb
    B, H, T, D = 1, 2, 11, 6
    V = torch.randn(B, H, T, D, generator=torch.Generator().manual_seed(72), dtype=F64)
    _, protos = orc.build_planes_protos(D, Kb, L)
    out = orc.race_module_ref(V, V, V, torch.zeros(D, L * Kb), protos, L, Kb, eps=eps)
    t = torch.arange(T, dtype=F64).view(1, 1, T, 1)
    known = L * V.cumsum(2) / (t + 1 + R * eps)
    assert (out - known).abs().max().item() < 1e-13


def test_prefix_ref_t1_closed_form():
    g = torch.Generator().manual_seed(1)
    pk, pq = softmax_probs(3, 1, 2, 4, g), softmax_probs(3, 1, 2, 4, g)
    v = torch.randn(3, 1, 4, generator=g, dtype=F64)
    out, _, _ = orc.race_prefix_ref(pk, pq, v, 1e-6)
    known = (pq * pk / (pk + 1e-6)).sum(-1, keepdim=True) * v
    assert (out - known).abs().max().item() < 1e-14


def test_gradcheck_prefix_and_module():
    g = torch.Generator().manual_seed(2)
    pk = softmax_probs(1, 5, 2, 4, g).requires_grad_()
    pq = softmax_probs(1, 5, 2, 4, g).requires_grad_()
    v = torch.randn(1, 5, 3, generator=g, dtype=F64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda a, b, c: orc.race_prefix_ref(a, b, c, 1e-3)[0], (pk, pq, v))
    planes_T, protos = orc.build_planes_protos(6, 2, 2, seed=4)
    Q, K, V = (torch.randn(1, 2, 4, 6, generator=g, dtype=F64, requires_grad=True) for _ in range(3))
    assert torch.autograd.gradcheck(
        lambda q, k, x: orc.race_module_ref(q, k, x, planes_T, protos, 2, 2, scale=1.0), (Q, K, V))


# ---------------------------------------------------------------- C restatements
def test_c_streaming_fwd_bwd_equal_autograd():
    g = torch.Generator().manual_seed(3)
    N, T, L, R, D, eps = 3, 40, 2, 8, 7, 1e-6
    pk, pq = softmax_probs(N, T, L, R, g), softmax_probs(N, T, L, R, g)
    v = torch.randn(N, T, D, generator=g, dtype=F64)
    go = torch.randn(N, T, D, generator=g, dtype=F64)
    a, b, c = (x.clone().requires_grad_() for x in (pk, pq, v))
    out, A, B = orc.race_prefix_ref(a, b, c, eps)
    (out * go).sum().backward()
    o2, A2, B2 = oracle_c.race_fwd(pk, pq, v, eps)
    assert orc.relerr(o2, out) < 1e-13 and orc.relerr(A2, A) < 1e-13 and orc.relerr(B2, B) < 1e-13
    gpk, gpq, gv = oracle_c.race_bwd(pk, pq, v, go, eps)
    assert orc.relerr(gpk, a.grad) < 1e-12
    assert orc.relerr(gpq, b.grad) < 1e-12
    assert orc.relerr(gv, c.grad) < 1e-12


def test_c_windows_equal_streaming_fwd_bwd():
    """orc_race_windows (buckets split over threads, outputs on windows) equals the full
    streaming C forward/backward on every window, including the first and last token."""
    g = torch.Generator().manual_seed(5)
    T, L, R, D, eps = 700, 3, 8, 9, 1e-6
    pk, pq = softmax_probs(1, T, L, R, g)[0], torch.rand(T, L * R, generator=g, dtype=F64)
    v = torch.randn(T, D, generator=g, dtype=F64)
    go = torch.randn(T, D, generator=g, dtype=F64)
    out, _, _ = oracle_c.race_fwd(pk[None], pq[None], v[None], eps)
    gpk, gpq, gv = oracle_c.race_bwd(pk[None], pq[None], v[None], go[None], eps)
    wins, wl = [0, 301, T - 33], 33
    o, a, b, c = oracle_c.race_windows(pk, pq, v, go, eps, wins, wl)
    of = oracle_c.race_windows(pk, pq, v, None, eps, wins, wl)
    for i, w in enumerate(wins):
        assert orc.relerr(o[i], out[0, w:w + wl]) < 1e-13 and torch.equal(of[i], o[i])
        assert orc.relerr(a[i], gpk[0, w:w + wl]) < 1e-12
        assert orc.relerr(b[i], gpq[0, w:w + wl]) < 1e-12
        assert orc.relerr(c[i], gv[0, w:w + wl]) < 1e-12
    with pytest.raises(ValueError):
        oracle_c.race_windows(pk, pq, v, None, eps, [0, 20], 33)  # overlapping windows


def test_c_windows_carried_state_is_the_prefix():
    """A window of [t0, T) scanned from the prefix state (A, B) of [0, t0) equals the same
    window of the whole sequence (the late-window check of the long-context sweep)."""
    g = torch.Generator().manual_seed(6)
    T, t0, S, D, eps = 900, 611, 16, 5, 1e-6
    pk, pq = softmax_probs(1, T, 2, 8, g)[0], softmax_probs(1, T, 2, 8, g)[0]
    v = torch.randn(T, D, generator=g, dtype=F64)
    out, _, _ = oracle_c.race_fwd(pk[None], pq[None], v[None], eps)
    A0 = pk[:t0].sum(0)
    B0 = pk[:t0].T @ v[:t0]
    o = oracle_c.race_windows(pk[t0:], pq[t0:], v[t0:], None, eps, [0, 100, T - t0 - 20], 20, A0, B0)
    for i, w in enumerate([0, 100, T - t0 - 20]):
        assert orc.relerr(o[i], out[0, t0 + w:t0 + w + 20]) < 1e-13


def test_group_windows_and_prefix_state_equal_layer_oracle():
    """tests/race_ref.oracle_group_windows (the full-size GPU tests' reference) equals the whole-
    sequence layer oracle on its windows, grouped-query heads included, and oracle_prefix_state
    equals race_prefix_ref's final state."""
    import sys
    sys.path.insert(0, os.path.dirname(__file__))
    from race_ref import oracle_group_windows, oracle_layer, oracle_prefix_state
    g = torch.Generator().manual_seed(8)
    B, Hq, Hkv, T, D, L, Kb, scale, eps = 2, 4, 2, 300, 16, 2, 3, 2.5, 1e-6
    q, k, v, go = (torch.randn(B, h, T, D, generator=g) for h in (Hq, Hkv, Hkv, Hq))
    planes_T, protos = orc.build_planes_protos(D, Kb, L, seed=3)
    ref = oracle_layer(q, k, v, planes_T, L, Kb, scale, eps, go)
    wins, wl = [0, 150, T - 20], 20
    for b, hk in ((0, 0), (1, 1)):
        out, dq, dk, dv = oracle_group_windows(q, k, v, go, planes_T, L, Kb, scale, eps, b, hk, wins, wl)
        for i, w in enumerate(wins):
            for gi in range(Hq // Hkv):
                h = hk * (Hq // Hkv) + gi
                assert orc.relerr(out[gi, i], ref[0][b, h, w:w + wl]) < 1e-12
                assert orc.relerr(dq[gi, i], ref[1][b, h, w:w + wl]) < 1e-10
            assert orc.relerr(dk[i], ref[2][b, hk, w:w + wl]) < 1e-10
            assert orc.relerr(dv[i], ref[3][b, hk, w:w + wl]) < 1e-10
    A, Bst = oracle_prefix_state(k[1, 0], v[1, 0], planes_T, L, Kb, scale, chunk=128)
    pK, _, V2, _ = orc.soft_hash_probs(k[1:, :1], k[1:, :1], v[1:, :1], planes_T, protos, L, Kb, scale=scale)
    _, A_ref, B_ref = orc.race_prefix_ref(pK, pK, V2)
    assert orc.relerr(A, A_ref[0]) < 1e-12 and orc.relerr(Bst, B_ref[0]) < 1e-12


def test_segment_windows_equal_layer_oracle():
    """tests/race_ref.oracle_segment_windows (the long-context sweep's reference: prefix state of
    [0, t0), then the streaming oracle over [t0, t1)) equals the whole-sequence layer oracle: out,
    dq, dk, dv on windows of a segment that runs to the end, and out, dq on a segment that stops
    early (dk, dv there lack the later tokens' suffix sums and are not claimed)."""
    import sys
    sys.path.insert(0, os.path.dirname(__file__))
    from race_ref import oracle_layer, oracle_segment_windows
    g = torch.Generator().manual_seed(9)
    B, H, T, D, L, Kb, scale, eps = 1, 3, 400, 16, 2, 3, 2.5, 1e-6
    q, k, v, go = (torch.randn(B, H, T, D, generator=g) for _ in range(4))
    planes_T, _ = orc.build_planes_protos(D, Kb, L, seed=4)
    ref = oracle_layer(q, k, v, planes_T, L, Kb, scale, eps, go)
    h, wl = 2, 16
    res = oracle_segment_windows(q, k, v, go, planes_T, L, Kb, scale, eps, 0, h, 250, T, [260, T - wl], wl)
    for r, full in zip(res, ref):
        for i, w in enumerate([260, T - wl]):
            assert orc.relerr(r[i], full[0, h, w:w + wl]) < 1e-10
    res = oracle_segment_windows(q, k, v, go, planes_T, L, Kb, scale, eps, 0, h, 100, 100 + wl, [100], wl)
    for r, full in zip(res[:2], ref[:2]):
        assert orc.relerr(r[0], full[0, h, 100:100 + wl]) < 1e-10
    assert orc.relerr(res[2][0], ref[2][0, h, 100:100 + wl]) > 1e-3  # the missing suffix shows
    out0 = oracle_segment_windows(q, k, v, None, planes_T, L, Kb, scale, eps, 0, h, 0, 40, [0], wl)
    assert orc.relerr(out0[0], ref[0][0, h, :wl]) < 1e-12


@pytest.mark.parametrize("NS,T,D", [(1, 1, 1), (4, 1, 8), (8, 16, 32), (16, 512, 64)])
def test_c_prefix_mean_flat(NS, T, D):
    """kernels/cpu/test_cpu_kernels.py:49-53 sweep: C restatement vs fp64 cumsum."""
    g = torch.Generator().manual_seed(NS + T)
    w = torch.rand(NS, T, generator=g)
    v = torch.randn(NS, T, D, generator=g)
    E = oracle_c.prefix_mean_flat(w, v, 1e-6)
    ref = (w.double().unsqueeze(-1) * v.double()).cumsum(1) / (w.double().cumsum(1).unsqueeze(-1) + 1e-6)
    assert orc.relerr(E, ref) < 1e-6
    wr = w.double().requires_grad_()
    vr = v.double().requires_grad_()
    gE = torch.randn(NS, T, D, generator=g)
    ((wr.unsqueeze(-1) * vr).cumsum(1) / (wr.cumsum(1).unsqueeze(-1) + 1e-6) * gE.double()).sum().backward()
    gW, gV = oracle_c.prefix_mean_flat_bw(w, v, gE, 1e-6)
    assert orc.relerr(gW, wr.grad) < 1e-5 and orc.relerr(gV, vr.grad) < 1e-5


def test_c_restatement_matches_compiled_reference():
    ext = oracle_c.ref_ext()
    if ext is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    g = torch.Generator().manual_seed(9)
    w = torch.rand(6, 300, generator=g)
    v = torch.randn(6, 300, 24, generator=g)
    gE = torch.randn(6, 300, 24, generator=g)
    assert torch.equal(ext.race_prefix_mean_flat(w, v, 1e-6), oracle_c.prefix_mean_flat(w, v, 1e-6))
    r_gw, r_gv = ext.race_prefix_mean_flat_bw(w, v, gE, 1e-6)
    o_gw, o_gv = oracle_c.prefix_mean_flat_bw(w, v, gE, 1e-6)
    assert torch.equal(r_gw, o_gw) and torch.equal(r_gv, o_gv)


def test_cpu_port_matches_oracle():
    """scaling/test_race_cpu_composite.py sweep, against the fp64 oracle."""
    g = torch.Generator().manual_seed(0)
    for (N, T, S, D) in [(2, 8, 6, 8), (4, 64, 24, 32)]:
        pk = torch.rand(N, T, S, generator=g)
        pq = torch.rand(N, T, S, generator=g)
        v = torch.randn(N, T, D, generator=g)
        go = torch.randn(N, T, D, generator=g)
        a, b, c = (x.clone().requires_grad_() for x in (pk, pq, v))
        out = race_cpu_port.RaceCausalCPUFn.apply(a, b, c, 1e-6)
        (out * go).sum().backward()
        ref = oracle_c.race_fwd(pk, pq, v, 1e-6)[0]
        gk, gq, gv = oracle_c.race_bwd(pk, pq, v, go, 1e-6)
        assert orc.relerr(out, ref) < 1e-4
        assert orc.relerr(a.grad, gk) < 1e-3 and orc.relerr(b.grad, gq) < 1e-3 and orc.relerr(c.grad, gv) < 1e-3


# ----------------------------------------------------------------------------- a11
def test_decode_ref_equals_module_position():
    g = torch.Generator().manual_seed(4)
    B, H, T, D, L, Kb = 2, 2, 6, 16, 2, 3
    planes_T, protos = orc.build_planes_protos(D, Kb, L, seed=0)
    Q, K, V = (torch.randn(B, H, T + 1, D, generator=g, dtype=F64) for _ in range(3))
    full = orc.race_module_ref(Q, K, V, planes_T, protos, L, Kb)
    out, A, Bst = orc.decode_ref(K[:, :, :T], V[:, :, :T], Q[:, :, T], K[:, :, T], V[:, :, T],
                                 planes_T, L, Kb)
    assert (out - full[:, :, T]).abs().max().item() < 1e-13


def test_gqa_ref_is_repeated_kv():
    g = torch.Generator().manual_seed(5)
    B, Hq, Hkv, T, D, L, Kb = 1, 4, 2, 5, 8, 2, 2
    planes_T, protos = orc.build_planes_protos(D, Kb, L, seed=0)
    Q = torch.randn(B, Hq, T, D, generator=g, dtype=F64)
    K, V = (torch.randn(B, Hkv, T, D, generator=g, dtype=F64) for _ in range(2))
    out = orc.race_gqa_ref(Q, K, V, planes_T, L, Kb)
    for h in range(Hq):
        one = orc.race_module_ref(Q[:, h:h + 1], K[:, h // 2:h // 2 + 1], V[:, h // 2:h // 2 + 1],
                                  planes_T, protos, L, Kb)
        assert (out[:, h:h + 1] - one).abs().max().item() < 1e-14


# ------------------------------------------------------------------ non-causal restatement
def _nc_inputs(N, T, S, D, seed):
    g = torch.Generator().manual_seed(seed)
    pk = torch.softmax(torch.randn(N, T, S, generator=g, dtype=torch.float64), -1)
    pq = torch.softmax(torch.randn(N, T, S, generator=g, dtype=torch.float64), -1)
    v = torch.randn(N, T, D, generator=g, dtype=torch.float64)
    return pk, pq, v


def test_noncausal_matches_brute_force():
    pk, pq, v = _nc_inputs(2, 9, 6, 5, 0)
    assert torch.allclose(orc.race_noncausal_ref(pk, pq, v), orc.race_noncausal_brute(pk, pq, v),
                          rtol=1e-12, atol=1e-12)


def test_noncausal_last_row_is_causal_last_row():
    pk, pq, v = _nc_inputs(3, 40, 16, 8, 1)
    nc = orc.race_noncausal_ref(pk, pq, v)
    ca, _, _ = orc.race_prefix_ref(pk, pq, v)
    assert torch.allclose(nc[:, -1], ca[:, -1], rtol=1e-12, atol=1e-12)
    assert not torch.allclose(nc[:, 0], ca[:, 0])  # earlier rows see the whole sequence


def test_noncausal_uniform_hash_closed_form():
    B, H, T, D, L, K, eps = 1, 2, 50, 8, 3, 2, 1e-3
    planes = torch.zeros(D, L * K, dtype=torch.float64)
    _, protos = orc.build_planes_protos(D, K, L)
    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(B, H, T, D, generator=g, dtype=torch.float64) for _ in range(3))
    pk, pq, v2, _ = orc.soft_hash_probs(q, k, v, planes, protos, L, K)
    out = orc.race_noncausal_ref(pk, pq, v2, eps)
    R = 1 << K
    want = L * v2.sum(1, keepdim=True) / (T + R * eps)
    assert torch.allclose(out, want.expand_as(out), rtol=1e-12, atol=1e-12)


def test_noncausal_single_token_closed_form():
    pk, pq, v = _nc_inputs(2, 1, 12, 4, 3)
    eps = 1e-2
    want = (pq * pk / (pk + eps)).sum(-1, keepdim=True) * v
    assert torch.allclose(orc.race_noncausal_ref(pk, pq, v, eps), want, rtol=1e-12, atol=1e-12)


def test_noncausal_gradcheck():
    pk, pq, v = _nc_inputs(1, 5, 4, 3, 4)
    for x in (pk, pq, v):
        x.requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b, c: orc.race_noncausal_ref(a, b, c, 1e-3), (pk, pq, v))


def test_batched_ace_nc_temperature_gradcheck():
    g = torch.Generator().manual_seed(5)
    M, B, T, H, dk, L, K = 2, 1, 6, 2, 4, 2, 2
    Kh, Vh, Qh = (torch.randn(M, B, T, H, dk, generator=g, dtype=torch.float64) for _ in range(3))
    planes = torch.randn(M, dk, L * K, generator=g, dtype=torch.float64)
    _, protos = orc.build_planes_protos(dk, K, L)
    lt = torch.tensor(0.3, dtype=torch.float64, requires_grad=True)
    Kh.requires_grad_(True)
    f = lambda t, kk: orc.batched_ace_nc_ref(kk, Vh, Qh, planes, protos, L, K, False, t)
    assert torch.autograd.gradcheck(f, (lt, Kh))
    # shared planes equal per-member planes when every member gets the same matrix
    shared = planes[0]
    a = orc.batched_ace_nc_ref(Kh, Vh, Qh, shared, protos, L, K, True, lt)
    b = orc.batched_ace_nc_ref(Kh, Vh, Qh, shared.expand(M, -1, -1), protos, L, K, False, lt)
    assert torch.allclose(a, b, rtol=1e-12, atol=1e-12)


def test_batched_ace_nc_distinct_member_planes():
    """Per-member planes with a DIFFERENT matrix for every member: member m of
    batched_ace_nc_ref equals race_noncausal_ref on the probabilities of member m's own
    [B,H,T,dk] slice hashed with planes[m] (so a wrong member-to-planes mapping fails), and the
    [M,B,T,H,dk] output layout holds it at [m, :, t, h]."""
    g = torch.Generator().manual_seed(9)
    M, B, T, H, dk, L, K = 3, 2, 7, 2, 8, 2, 3
    Kh, Vh, Qh = (torch.randn(M, B, T, H, dk, generator=g, dtype=F64) for _ in range(3))
    planes = torch.randn(M, dk, L * K, generator=g, dtype=F64)
    _, protos = orc.build_planes_protos(dk, K, L)
    lt = torch.tensor(-0.4, dtype=F64)
    out = orc.batched_ace_nc_ref(Kh, Vh, Qh, planes, protos, L, K, False, lt)
    scale = float(lt.exp())
    for m in range(M):
        q, k, v = (X[m].permute(0, 2, 1, 3) for X in (Qh, Kh, Vh))  # [B,H,T,dk]
        pK, pQ, V2, N = orc.soft_hash_probs(q, k, v, planes[m], protos, L, K, scale=scale)
        ref = orc.race_noncausal_ref(pK, pQ, V2).view(B, H, T, dk).permute(0, 2, 1, 3)
        assert torch.allclose(out[m], ref, rtol=1e-12, atol=1e-12), m
        for m2 in range(M):  # another member's planes give a different answer
            if m2 != m:
                pK2, pQ2, _, _ = orc.soft_hash_probs(q, k, v, planes[m2], protos, L, K, scale=scale)
                other = orc.race_noncausal_ref(pK2, pQ2, V2).view(B, H, T, dk).permute(0, 2, 1, 3)
                assert (other - out[m]).abs().max().item() > 1e-6


# ------------------------------------------------------------------ causal linear attention
def _lin_inputs(N, H, L, E, M, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(N, H, L, E, generator=g), torch.randn(N, H, L, E, generator=g),
            torch.randn(N, H, L, M, generator=g))


def test_causal_linear_matches_brute_force():
    Q, K, V = _lin_inputs(2, 2, 9, 4, 3, 0)
    assert torch.allclose(orc.causal_linear_ref(Q, K, V), orc.causal_linear_brute(Q, K, V), rtol=1e-12, atol=1e-12)


def test_causal_linear_gradcheck():
    Q, K, V = (x.double().requires_grad_(True) for x in _lin_inputs(1, 1, 5, 3, 2, 1))
    assert torch.autograd.gradcheck(orc.causal_linear_ref, (Q, K, V))


def test_causal_linear_matches_compiled_reference():
    """The reference's own linear_pref.cpp (compiled into oracle/_ref from its source)."""
    from oracle import oracle_c
    ext = oracle_c.ref_linear_ext()
    if ext is None:
        pytest.skip("oracle/_ref/linear_pref_ref.so not built (reference tree absent)")
    for (N, H, L, E, M) in [(1, 1, 1, 4, 4), (2, 2, 16, 8, 8), (2, 4, 256, 32, 32)]:
        Q, K, V = _lin_inputs(N, H, L, E, M, L)
        out = torch.zeros(N, H, L, M)
        ext.causal_dot_product(Q.contiguous(), K.contiguous(), V.contiguous(), out)
        assert orc.relerr(out, orc.causal_linear_ref(Q, K, V)) < 1e-5
        g = torch.randn(N, H, L, M)
        gQ, gK, gV = torch.zeros_like(Q), torch.zeros_like(K), torch.zeros_like(V)
        ext.causal_dot_backward(Q, K, V, g, gQ, gK, gV)
        q1, k1, v1 = (x.double().requires_grad_(True) for x in (Q, K, V))
        (orc.causal_linear_ref(q1, k1, v1) * g.double()).sum().backward()
        for a, b in ((gQ, q1.grad), (gK, k1.grad), (gV, v1.grad)):
            assert orc.relerr(a, b) < 1e-5
