"""Fused bf16 q/k/v kernels, soft-hash kernel, modules and decode on the GPU,
against the fp64 oracle (2e-2 for bf16, 1e-4 for fp32,
max-normalised error as scaling/test_kernels.py:30-31)."""
import math

import numpy as np
import pytest
import torch

from oracle import race_oracle as orc
from race_ref import bf16_planes, check, oracle_layer

pytestmark = pytest.mark.gpu

EPS = 1e-6
BF16_TOL = 2e-2


def qkv(B, Hq, Hkv, T, D, seed, dev, std=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, Hq, T, D, generator=g) * std).to(torch.bfloat16)
    k = (torch.randn(B, Hkv, T, D, generator=g) * std).to(torch.bfloat16)
    v = (torch.randn(B, Hkv, T, D, generator=g) * std).to(torch.bfloat16)
    go = torch.randn(B, Hq, T, D, generator=g).to(torch.bfloat16)
    return q.to(dev), k.to(dev), v.to(dev), go.to(dev)


FUSED_CASES = [  # B, Hq, Hkv, T, D, L, K, scale
    (1, 2, 2, 256, 64, 8, 4, None),
    (1, 2, 2, 1000, 64, 16, 4, None),     # S = 256: two bucket tiles
    (2, 2, 2, 333, 128, 3, 3, None),      # nanochat default L=3, K=3 at head dim 128
    (1, 4, 2, 777, 64, 8, 4, None),       # grouped-query heads
    (1, 2, 2, 513, 64, 4, 2, 1.0),        # K=2, temperature-1 scale
    (1, 1, 1, 4096, 64, 8, 4, None),
    (1, 2, 1, 300, 128, 4, 4, 1.0),
    (1, 2, 2, 1, 64, 8, 4, None),         # a single token
    (2, 2, 2, 31, 64, 8, 4, None),        # shorter than one 32-token sub-chunk
    (1, 8, 2, 200, 64, 16, 4, None),      # grouped-query heads with two bucket tiles
    (1, 8, 1, 97, 128, 16, 3, 1.0),       # 8 query heads per kv head, K=3 at 128 buckets
    (1, 2, 2, 600, 64, 4, 4, None),       # S = 64 at head dim 64: 64-bucket tile
    (1, 2, 2, 700, 64, 16, 3, None),      # K=3 at 128 buckets, head dim 64
    (1, 2, 2, 400, 64, 32, 2, 1.0),       # K=2 at 128 buckets
    (2, 6, 2, 450, 64, 8, 3, None),       # S = 64, K=3, grouped-query heads
    (1, 3, 1, 2000, 64, 16, 4, None),     # grouped-query heads, many sub-chunks per block
]


@pytest.mark.parametrize("case", FUSED_CASES)
def test_fused_forward_backward(dev, case):
    from race_attention_amd import build_planes_protos, race_causal_attention
    B, Hq, Hkv, T, D, L, Kb, scale = case
    print("fused case", case, flush=True)
    scale = math.sqrt(D) if scale is None else scale
    planes_T, _ = build_planes_protos(D, Kb, L, 1, device=dev, seed=0)
    q, k, v, go = qkv(B, Hq, Hkv, T, D, seed=T + D, dev=dev)
    qx, kx, vx = (x.clone().requires_grad_(True) for x in (q, k, v))
    out = race_causal_attention(qx, kx, vx, planes_T, L, Kb, scale=scale, eps=EPS)
    out.backward(go)
    ref_out, ref_dq, ref_dk, ref_dv = oracle_layer(q, k, v, bf16_planes(planes_T), L, Kb, scale, EPS, go)
    check("out", out, ref_out, BF16_TOL)
    check("dq", qx.grad, ref_dq, BF16_TOL)
    if T >= 64:
        check("dk", kx.grad, ref_dk, BF16_TOL)
    else:
        # For a sequence's first tokens dL/dpK is a difference of two nearly equal terms: at
        # t = 0, gA = -(go.v) pQ pK/(pK+eps)^2 against (go.v) pQ/(pK+eps) from the state, which
        # cancel to (go.v) pQ eps/(pK+eps)^2 ~ 1e-6. The bf16 path forms both terms from
        # bf16-rounded operands, so there dk carries bf16 noise of O(1) terms while the exact
        # dk is ~0 and the per-tensor normalisation degenerates. A sequence shorter than two
        # sub-chunks is checked against the common scale of the three input gradients.
        gscale = max(ref_dq.abs().max(), ref_dk.abs().max(), ref_dv.abs().max()).item()
        err = (kx.grad.double().cpu() - ref_dk).abs().max().item()
        assert err <= BF16_TOL * gscale, f"dk: max error {err:.3e} > {BF16_TOL:.0e} x gradient scale {gscale:.3e}"
    check("dv", vx.grad, ref_dv, BF16_TOL)


@pytest.mark.parametrize("block", [32, 64, 96, 160])
def test_fused_headline_shape_short_blocks(dev, block):
    """The headline head shape (one query head per kv head, D=64, L=8, K=4, bf16) with blocks of
    1, 2, 3 and 5 sub-chunks and a ragged last one: the wave-specialised backward totals kernel's
    prologue, its loop unrolled by two and the trailing odd sub-chunk, against the fp64 oracle."""
    from race_attention_amd import build_planes_protos, race_causal_attention
    B, H, T, D, L, Kb = 1, 2, 333, 64, 8, 4
    print("headline shape, block", block, flush=True)
    scale = math.sqrt(D)
    planes_T, _ = build_planes_protos(D, Kb, L, 1, device=dev, seed=3)
    q, k, v, go = qkv(B, H, H, T, D, seed=block, dev=dev)
    qx, kx, vx = (x.clone().requires_grad_(True) for x in (q, k, v))
    out = race_causal_attention(qx, kx, vx, planes_T, L, Kb, scale=scale, eps=EPS, block=block)
    out.backward(go)
    ref_out, ref_dq, ref_dk, ref_dv = oracle_layer(q, k, v, bf16_planes(planes_T), L, Kb, scale, EPS, go)
    check("out", out, ref_out, BF16_TOL)
    check("dq", qx.grad, ref_dq, BF16_TOL)
    check("dk", kx.grad, ref_dk, BF16_TOL)
    check("dv", vx.grad, ref_dv, BF16_TOL)


def test_fused_block_invariance_and_determinism(dev):
    from race_attention_amd import build_planes_protos, race_causal_attention
    planes_T, _ = build_planes_protos(64, 4, 8, 1, device=dev, seed=0)
    q, k, v, _ = qkv(1, 2, 2, 2000, 64, seed=5, dev=dev)
    outs = [race_causal_attention(q, k, v, planes_T, 8, 4, block=b, out_dtype=torch.float32)
            for b in (0, 128, 512, 2048)]
    for o in outs[1:]:
        check("block invariance", o, outs[0], 1e-3)
    again = race_causal_attention(q, k, v, planes_T, 8, 4, out_dtype=torch.float32)
    assert torch.equal(again, outs[0]), "fused forward is not bitwise deterministic"


def test_fused_backward_block_invariance_and_determinism(dev):
    """dq/dk/dv do not depend on the block decomposition (1 .. 16 blocks: the reverse block scan
    of the suffix states) beyond fp32 rounding, and repeat bitwise."""
    from race_attention_amd import build_planes_protos, race_causal_attention
    planes_T, _ = build_planes_protos(64, 4, 8, 1, device=dev, seed=2)
    q, k, v, go = qkv(1, 2, 2, 2000, 64, seed=6, dev=dev)

    def grads(block):
        xs = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]
        race_causal_attention(*xs, planes_T, 8, 4, block=block, out_dtype=torch.float32).backward(go.float())
        return [x.grad.float() for x in xs]

    ref = grads(0)
    for b in (128, 512, 2048):
        for name, g, r in zip(("dq", "dk", "dv"), grads(b), ref):
            check(f"{name} block={b}", g, r, 1e-2)
    for g, r in zip(grads(0), ref):
        assert torch.equal(g, r), "fused backward is not bitwise deterministic"


def test_fused_strided_views(dev):
    """[B,T,H,D] storage viewed as [B,H,T,D] (the nanochat layout) needs no copy."""
    from race_attention_amd import build_planes_protos, race_causal_attention
    planes_T, _ = build_planes_protos(64, 4, 8, 1, device=dev, seed=1)
    q, k, v, _ = qkv(2, 4, 4, 200, 64, seed=9, dev=dev)
    qt, kt, vt = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (q, k, v))
    a = race_causal_attention(q, k, v, planes_T, 8, 4, out_dtype=torch.float32)
    b = race_causal_attention(qt, kt, vt, planes_T, 8, 4, out_dtype=torch.float32)
    assert torch.equal(a, b)


def test_soft_hash_probs_fp32(dev):
    from race_attention_amd import build_planes_protos, soft_hash_probs
    # D = 130: rows not a multiple of 4 (element-wise x loads, zero-padded LDS rows) and the backward
    # compiled for D <= 256; D = 256: the largest head dim
    for (L, Kb, D, M, share) in [(2, 2, 16, 1, True), (8, 4, 64, 1, True), (3, 3, 128, 2, True),
                                 (4, 2, 32, 3, False), (2, 3, 130, 1, True), (4, 4, 256, 2, False)]:
        planes_T, protos_T = build_planes_protos(D, Kb, L, M, device=dev, share_planes=share, seed=2)
        g = torch.Generator().manual_seed(D)
        Q, K, V = (torch.randn(2, 3, 37, D, generator=g) for _ in range(3))
        Qd, Kd, Vd = (x.to(dev).requires_grad_(True) for x in (Q, K, V))
        pK, pQ, V2, N = soft_hash_probs(Qd, Kd, Vd, planes_T, protos_T, L, Kb, M, share)
        rK, rQ, rV, rN = orc.soft_hash_probs(Q, K, V, planes_T.cpu(), protos_T.cpu(), L, Kb, M, share)
        assert N == rN and pK.shape == rK.shape
        check("probsK", pK, rK, 1e-5)
        check("probsQ", pQ, rQ, 1e-5)
        gk = torch.randn(pK.shape, generator=g)
        gq = torch.randn(pQ.shape, generator=g)
        torch.autograd.backward([pK, pQ], [gk.to(dev), gq.to(dev)])
        Q64, K64 = (x.double().requires_grad_(True) for x in (Q, K))
        r2K, r2Q, _, _ = orc.soft_hash_probs(Q64, K64, V, planes_T.cpu(), protos_T.cpu(), L, Kb, M, share)
        torch.autograd.backward([r2K, r2Q], [gk.double(), gq.double()])
        check("dQ", Qd.grad, Q64.grad, 1e-4)
        check("dK", Kd.grad, K64.grad, 1e-4)


@pytest.mark.parametrize("B,H,T,D,L,Kb,M,share", [(4, 8, 4141, 64, 4, 3, 2, False), (4, 8, 16389, 64, 2, 2, 1, True),
                                                   (1, 8, 524365, 16, 3, 3, 1, True)])
def test_soft_hash_probs_multi_tile(dev, B, H, T, D, L, Kb, M, share):
    """Enough token tiles (32 tokens for the FMA kernels, 64 for the matrix-core ones) that each
    soft-hash workgroup walks several of them (1 to 32 per workgroup here), with a ragged last tile
    and a last workgroup that holds fewer tiles."""
    from race_attention_amd import build_planes_protos, soft_hash_probs
    print(f"case B={B} H={H} T={T} D={D} L={L} K={Kb} M={M} share={share}", flush=True)
    planes_T, protos_T = build_planes_protos(D, Kb, L, M, device=dev, share_planes=share, seed=4)
    g = torch.Generator().manual_seed(T)
    Q, K, V = (torch.randn(B, H, T, D, generator=g) for _ in range(3))
    Qd, Kd, Vd = (x.to(dev).requires_grad_(True) for x in (Q, K, V))
    pK, pQ, V2, N = soft_hash_probs(Qd, Kd, Vd, planes_T, protos_T, L, Kb, M, share)
    Q64, K64 = (x.double().requires_grad_(True) for x in (Q, K))
    rK, rQ, _, rN = orc.soft_hash_probs(Q64, K64, V, planes_T.cpu(), protos_T.cpu(), L, Kb, M, share)
    assert N == rN and pK.shape == rK.shape
    check("probsK", pK, rK.detach(), 1e-5)
    check("probsQ", pQ, rQ.detach(), 1e-5)
    gk = torch.randn(pK.shape, generator=g)
    gq = torch.randn(pQ.shape, generator=g)
    torch.autograd.backward([pK, pQ], [gk.to(dev), gq.to(dev)])
    torch.autograd.backward([rK, rQ], [gk.double(), gq.double()])
    check("dQ", Qd.grad, Q64.grad, 1e-4)
    check("dK", Kd.grad, K64.grad, 1e-4)


def test_soft_hash_probs_golden(dev):
    """Against the reference's own outputs (tests/golden, written by scaling/race_common.py)."""
    from race_attention_amd import soft_hash_probs
    import os
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "soft_hash_golden.npz"))
    for i in range(6):
        B, H, T, D, L, Kb, seed, is_bf16 = (int(x) for x in z[f"c{i}_meta"])
        dt = torch.bfloat16 if is_bf16 else torch.float32
        Q, K, V = (torch.from_numpy(z[f"c{i}_{n}"]).to(dev, dt) for n in "QKV")
        planes_T = torch.from_numpy(z[f"c{i}_planes_T"]).to(dev)
        protos_T = torch.from_numpy(z[f"c{i}_protos_T"]).to(dev)
        pK, pQ, _, _ = soft_hash_probs(Q, K, V, planes_T, protos_T, L, Kb, 1, True)
        tol = BF16_TOL if is_bf16 else 1e-5
        check(f"golden{i} K", pK, torch.from_numpy(z[f"c{i}_probsK"]), tol)
        check(f"golden{i} Q", pQ, torch.from_numpy(z[f"c{i}_probsQ"]), tol)


@pytest.mark.parametrize("H,T,D,L,Kb", [(4, 256, 64, 2, 2), (8, 1024, 128, 3, 3), (4, 2048, 96, 4, 4),
                                        (2, 512, 64, 8, 4)])
def test_module_e2e_fp32(dev, H, T, D, L, Kb):
    """scaling/test_kernels.py:107-129: RaceCausalCuda (fp32) against the fp64 layer, at the north
    star's fp32 bar 1e-4 for the gradients."""
    from race_attention_amd import RaceCausalCuda
    torch.manual_seed(H + T)
    Q, K, V = (torch.randn(1, H, T, D) for _ in range(3))
    m = RaceCausalCuda(D, Kb, L, 1, device=dev, seed=0)
    qc, kc, vc = (x.to(dev).requires_grad_(True) for x in (Q, K, V))
    oc = m(qc, kc, vc)
    go = torch.randn(oc.shape)
    oc.backward(go.to(dev))
    ref, dq, dk, dv = oracle_layer(Q, K, V, m.planes_T.cpu(), L, Kb, math.sqrt(D), EPS, go)
    assert oc.dtype == torch.float32
    check("e2e out", oc, ref, 2e-5)
    check("e2e gradQ", qc.grad, dq, 1e-4)  # north-star fp32 bar (the reference's e2e test: 2e-3)
    check("e2e gradK", kc.grad, dk, 1e-4)
    check("e2e gradV", vc.grad, dv, 1e-4)


def test_module_bf16_and_ensemble(dev):
    from race_attention_amd import RaceCausalCuda, RaceCumsumCausal
    m = RaceCausalCuda(64, 4, 8, 3, device=dev, seed=0)  # M=3 shared planes == M=1
    q, k, v, go = qkv(1, 2, 2, 300, 64, seed=3, dev=dev)
    out = m(q, k, v)
    assert out.dtype == torch.float32 and out.shape == q.shape
    ref = oracle_layer(q, k, v, bf16_planes(m.planes_T), 8, 4, 8.0, EPS)
    check("bf16 module", out, ref, BF16_TOL)
    mc = RaceCumsumCausal(64, 4, 8, 1, device=dev, seed=0)
    Q, K, V = (torch.randn(1, 2, 64, 64, device=dev) for _ in range(3))
    check("cumsum module vs scan", mc(Q, K, V), RaceCausalCuda(64, 4, 8, 1, device=dev, seed=0)(Q, K, V), 1e-5)


def test_batched_ace(dev):
    from race_attention_amd import BatchedACE
    torch.manual_seed(0)
    ace = BatchedACE(32, 3, 2, 2, device=dev, share_planes=True)
    M, B, T, H, dk = 2, 2, 50, 3, 32
    Khf, Vhf, Qhf = (torch.randn(M, B, T, H, dk, device=dev) for _ in range(3))
    out = ace(Khf, Vhf, Qhf)
    assert out.shape == (M, B, T, H, dk)
    ref = oracle_layer(Qhf.reshape(M * B, T, H, dk).transpose(1, 2), Khf.reshape(M * B, T, H, dk).transpose(1, 2),
                       Vhf.reshape(M * B, T, H, dk).transpose(1, 2), ace.planes_T.cpu(), 2, 3, math.sqrt(dk), EPS)
    check("BatchedACE", out, ref.transpose(1, 2).reshape(M, B, T, H, dk), 2e-5)
    un = BatchedACE(32, 3, 2, 2, device=dev, share_planes=False)
    out2 = un(Khf, Vhf, Qhf)
    for m in range(M):
        r = oracle_layer(Qhf[m].transpose(1, 2), Khf[m].transpose(1, 2), Vhf[m].transpose(1, 2),
                         un.planes_T[m].cpu(), 2, 3, math.sqrt(dk), EPS)
        check(f"BatchedACE unshared m={m}", out2[m], r.transpose(1, 2), 2e-5)


@pytest.mark.parametrize("G,D", [(4, 64), (1, 128), (2, 64), (3, 64), (6, 128), (8, 64)])
def test_decode_matches_forward(dev, G, D):
    """prefill T0 tokens, then decode steps: each step equals the full causal
    forward at that position (the reference's GPT.generate recomputation)."""
    from race_attention_amd import RaceDecodeState, build_planes_protos
    B, Hkv, T0, steps, L, Kb = 3, 2, 100, 5, 8, 4
    Hq = Hkv * G
    planes_T, _ = build_planes_protos(D, Kb, L, 1, device=dev, seed=4)
    q, k, v, _ = qkv(B, Hq, Hkv, T0 + steps, D, seed=G * 10 + D, dev=dev)
    st = RaceDecodeState(B, Hq, Hkv, D, L, Kb, planes_T, device=dev)
    pre = st.prefill(q[:, :, :T0], k[:, :, :T0], v[:, :, :T0], out_dtype=torch.float32)
    ref = oracle_layer(q, k, v, bf16_planes(planes_T), L, Kb, math.sqrt(D), EPS)
    check("prefill", pre, ref[:, :, :T0], BF16_TOL)
    for i in range(steps):
        t = T0 + i
        o = st.step(q[:, :, t], k[:, :, t], v[:, :, t])
        check(f"decode step {i}", o, ref[:, :, t], BF16_TOL)
    # the carried state equals the oracle's (A_final, B_final)
    kr = k.double().cpu().repeat_interleave(1, 1)
    _, protos = orc.build_planes_protos(D, Kb, L)
    pK, _, V2, _ = orc.soft_hash_probs(kr, kr, v.double().cpu(), bf16_planes(planes_T).cpu(), protos, L, Kb)
    _, A_ref, B_ref = orc.race_prefix_ref(pK, pK, V2)
    check("state A", st.A, A_ref, 1e-2)
    check("state B", st.Bs, B_ref, BF16_TOL)


def test_decode_fp32_from_zero(dev):
    from race_attention_amd import RaceDecodeState, build_planes_protos
    B, Hq, Hkv, D, L, Kb, T = 2, 4, 4, 64, 2, 3, 6
    planes_T, _ = build_planes_protos(D, Kb, L, 1, device=dev, seed=1)
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(B, H, T, D, generator=g) for H in (Hq, Hkv, Hkv))
    st = RaceDecodeState(B, Hq, Hkv, D, L, Kb, planes_T, device=dev)
    ref = oracle_layer(q, k, v, planes_T, L, Kb, math.sqrt(D), EPS)
    for t in range(T):
        o = st.step(q[:, :, t].to(dev), k[:, :, t].to(dev), v[:, :, t].to(dev))
        check(f"fp32 decode {t}", o, ref[:, :, t], 1e-4)
