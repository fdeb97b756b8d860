"""fp64 references for the GPU tests, built from the pinned oracle (oracle/).

oracle_op      fp64 streaming C forward/backward of the op-level scan
oracle_layer   fp64 soft-hash (torch autograd) + fp64 streaming C scan, chained:
               out, dq, dk, dv for q [B,Hq,T,D], k/v [B,Hkv,T,D] (GQA by repeat),
               with memory O(T*S) so long sequences stay checkable.
"""
import math

import torch

from oracle import oracle_c
from oracle import race_oracle as orc

F64 = torch.float64


def relerr(got, ref):
    return orc.relerr(got, ref)


def check(name, got, ref, tol, abs_floor=2e-5):
    """The reference's pass rule (scaling/test_kernels.py:38-51): relerr <= tol, or a
    tight absolute floor for genuinely near-zero references."""
    re = orc.relerr(got, ref)
    ma = orc.maxabs(got, ref)
    assert re <= tol or ma <= abs_floor, f"{name}: relerr {re:.3e} > {tol:.0e} (maxabs {ma:.3e})"
    return re


def make_probs(N, T, L, R, D, seed, dist="softmax"):
    """scaling/test_kernels.py:54-66 input distributions, fp64 on the CPU."""
    g = torch.Generator().manual_seed(seed)
    if dist in ("softmax", "sharp"):
        # "sharp": logits x4, probabilities from ~1e-7 to ~1 (temperature-1 soft-hash of N(0,1) rows
        # spans 2e-4 .. 0.8): tiny A at a sequence's first tokens, W = pQ/(A+eps) up to ~1e5
        sc = 4.0 if dist == "sharp" else 1.0
        pk = torch.softmax(sc * torch.randn(N, T, L, R, generator=g, dtype=F64), -1).reshape(N, T, L * R)
        pq = torch.softmax(sc * torch.randn(N, T, L, R, generator=g, dtype=F64), -1).reshape(N, T, L * R)
    else:
        pk = torch.rand(N, T, L * R, generator=g, dtype=F64)
        pq = torch.rand(N, T, L * R, generator=g, dtype=F64)
    v = torch.randn(N, T, D, generator=g, dtype=F64)
    go = torch.randn(N, T, D, generator=g, dtype=F64)
    return pk, pq, v, go


def oracle_op(pk, pq, v, go, eps):
    out, A, B = oracle_c.race_fwd(pk, pq, v, eps)
    gpk, gpq, gv = oracle_c.race_bwd(pk, pq, v, go, eps)
    return out, gpk, gpq, gv, A, B


def oracle_layer(q, k, v, planes_T, L, Kb, scale, eps, go=None):
    """fp64 out (and dq, dk, dv if go is given). Inputs may be bf16: they are taken
    at their exact values; planes are taken as given (round them to bf16 first to
    match a bf16 run, as the reference does at race_common.py:54)."""
    B, Hq, T, D = q.shape
    Hkv = k.shape[1]
    rep = Hq // Hkv
    q64 = q.detach().to("cpu", F64).requires_grad_(go is not None)
    k64 = k.detach().to("cpu", F64).requires_grad_(go is not None)
    v64 = v.detach().to("cpu", F64).requires_grad_(go is not None)
    kr = k64.repeat_interleave(rep, dim=1)
    vr = v64.repeat_interleave(rep, dim=1)
    _, protos = orc.build_planes_protos(D, Kb, L)
    pK, pQ, V2, N = orc.soft_hash_probs(q64, kr, vr, planes_T.detach().cpu().to(F64), protos, L, Kb,
                                        scale=scale)
    out, _, _ = oracle_c.race_fwd(pK.detach(), pQ.detach(), V2.detach(), eps)
    out = out.view(B, Hq, T, D)
    if go is None:
        return out
    g64 = go.detach().to("cpu", F64).reshape(N, T, D)
    gpk, gpq, gv = oracle_c.race_bwd(pK.detach(), pQ.detach(), V2.detach(), g64, eps)
    torch.autograd.backward([pK, pQ, V2], [gpk, gpq, gv])
    return out, q64.grad, k64.grad, v64.grad


def bf16_planes(planes_T):
    return planes_T.to(torch.bfloat16).float()


def default_scale(D):
    return math.sqrt(D)


def _stream_probs(x, planes_T, L, Kb, scale):
    """fp64 soft-hash probabilities [T, S] of one stream's rows x [T, D] (race_common.py:36-73)."""
    D = x.shape[-1]
    _, protos = orc.build_planes_protos(D, Kb, L)
    xs = x.reshape(1, 1, -1, D)
    p, _, _, _ = orc.soft_hash_probs(xs, xs, xs, planes_T.detach().cpu().to(F64), protos, L, Kb, scale=scale)
    return p[0]


def oracle_group_windows(q, k, v, go, planes_T, L, Kb, scale, eps, b, hk, wins, wlen):
    """fp64 reference of kv head `hk` of batch `b` and its query-head group on token windows
    [w, w + wlen) of an arbitrarily long sequence (q [B,Hq,T,D], k/v [B,Hkv,T,D], any dtype;
    their values are taken exactly). The whole stream is soft-hashed and scanned by the
    streaming C oracle (oracle_c.race_windows), so the backward's suffix sums cover every
    token; the soft-hash backward runs on the window rows only.
    Returns out, dq [G, nwin, wlen, D] (the group's query heads) and dk, dv [nwin, wlen, D],
    or only out when go is None."""
    G = q.shape[1] // k.shape[1]
    wins = sorted(int(w) for w in wins)
    idx = torch.cat([torch.arange(w, w + wlen) for w in wins])
    ks = k[b, hk].detach().to("cpu", F64)
    vs = v[b, hk].detach().to("cpu", F64)
    pK = _stream_probs(ks, planes_T, L, Kb, scale)
    outs, dqs = [], []
    gpk_sum, gv_sum = 0, 0
    for g in range(G):
        h = hk * G + g
        qs = q[b, h].detach().to("cpu", F64)
        pQ = _stream_probs(qs, planes_T, L, Kb, scale)
        gos = None if go is None else go[b, h].detach().to("cpu", F64)
        res = oracle_c.race_windows(pK, pQ, vs, gos, eps, wins, wlen)
        del pQ
        if go is None:
            outs.append(res)
            continue
        out_w, gpk_w, gpq_w, gv_w = res
        outs.append(out_w)
        qw = qs[idx].clone().requires_grad_(True)
        pqw = _stream_probs(qw, planes_T, L, Kb, scale)
        pqw.backward(gpq_w.reshape(-1, gpq_w.shape[-1]))
        dqs.append(qw.grad.view(len(wins), wlen, -1))
        gpk_sum = gpk_sum + gpk_w
        gv_sum = gv_sum + gv_w
    out = torch.stack(outs)
    if go is None:
        return out
    kw = ks[idx].clone().requires_grad_(True)
    pkw = _stream_probs(kw, planes_T, L, Kb, scale)
    pkw.backward(gpk_sum.reshape(-1, gpk_sum.shape[-1]))
    return out, torch.stack(dqs), kw.grad.view(len(wins), wlen, -1), gv_sum


def oracle_prefix_state(k_rows, v_rows, planes_T, L, Kb, scale, chunk=1 << 20):
    """fp64 bucket state (A [S], B [S, D]) after the given rows of one kv stream
    (race_prefix_ref's A_final / B_final, race_common.py:88-90), in chunks of `chunk` tokens."""
    A, Bst = None, None
    for c0 in range(0, k_rows.shape[0], chunk):
        kc = k_rows[c0:c0 + chunk].detach().to("cpu", F64)
        vc = v_rows[c0:c0 + chunk].detach().to("cpu", F64)
        p = _stream_probs(kc, planes_T, L, Kb, scale)
        a, bb = p.sum(0), p.T @ vc
        A = a if A is None else A + a
        Bst = bb if Bst is None else Bst + bb
    return A, Bst


def oracle_segment_windows(q, k, v, go, planes_T, L, Kb, scale, eps, b, h, t0, t1, wins, wlen):
    """fp64 reference of one (b, h) stream with one query head per kv head (q, k, v, go
    [B,H,T,D], any dtype, values taken exactly) on token windows inside the segment [t0, t1):
    the bucket state of tokens [0, t0) comes from oracle_prefix_state, then the streaming C oracle
    (oracle_c.race_windows) runs over [t0, t1) from it. out and dq need only the prefix, so they
    are exact for any t1; dk and dv need the suffix sums of every later token, so they are exact
    only when t1 = T (with go None only out is returned). `wins` are absolute window starts.
    Returns out, dq, dk, dv [nwin, wlen, D] fp64."""
    wins = sorted(int(w) for w in wins)
    assert all(t0 <= w and w + wlen <= t1 for w in wins), (t0, t1, wins)
    A0, B0 = oracle_prefix_state(k[b, h, :t0], v[b, h, :t0], planes_T, L, Kb, scale)
    ks = k[b, h, t0:t1].detach().to("cpu", F64)
    qs = q[b, h, t0:t1].detach().to("cpu", F64)
    vs = v[b, h, t0:t1].detach().to("cpu", F64)
    pK = _stream_probs(ks, planes_T, L, Kb, scale)
    pQ = _stream_probs(qs, planes_T, L, Kb, scale)
    rel = [w - t0 for w in wins]
    gos = None if go is None else go[b, h, t0:t1].detach().to("cpu", F64)
    res = oracle_c.race_windows(pK, pQ, vs, gos, eps, rel, wlen, A0, B0)
    del pK, pQ
    if go is None:
        return res
    out_w, gpk_w, gpq_w, gv_w = res
    idx = torch.cat([torch.arange(w, w + wlen) for w in rel])
    nw, S = len(wins), gpq_w.shape[-1]
    qw = qs[idx].clone().requires_grad_(True)
    _stream_probs(qw, planes_T, L, Kb, scale).backward(gpq_w.reshape(-1, S))
    kw = ks[idx].clone().requires_grad_(True)
    _stream_probs(kw, planes_T, L, Kb, scale).backward(gpk_w.reshape(-1, S))
    return out_w, qw.grad.view(nw, wlen, -1), kw.grad.view(nw, wlen, -1), gv_w


def qkv_blocks(T, Z, L, Kb, D=64, C=32, target=768):
    """The fused kernels' automatic block size and count (tokens per workgroup, as
    race_abi.cpp's qkv_geometry / resolve_block choose them) for Z = B*Hkv kv streams."""
    S = L << Kb
    st_max = 128 if D == 64 else 64
    st = next((x for x in (32, 64, 128) if st_max >= x >= S), st_max)
    n_st = -(-S // st)
    # the fused kernels (K = 2..4) launch one bucket tile at a time: ~target workgroups per tile
    if 2 <= Kb <= 4:
        n_st = 1
    nb = max(1, -(-target // (Z * n_st)))
    cb = max(4 * C, -(-(-(-T // nb)) // C) * C)
    cb = min(cb, -(-T // C) * C)
    return cb, -(-T // cb)


def fp32_formula_floor(pk, pq, v, go, eps, ref):
    """relerr against the fp64 gradients `ref` (gpK, gpQ, gV) of the reference formula itself
    evaluated in fp32: race_prefix_ref's cumsums (scaling/race_common.py:76-90) with torch
    autograd, the reference's own arithmetic. It measures the cancellation that fp32 cannot avoid
    (a sequence's first tokens: gpK = pQ <go, v> eps / (pK + eps)^2 from two O(1/pK) terms)."""
    xs = [x.float().clone().requires_grad_(True) for x in (pk, pq, v)]
    out, _, _ = orc.race_prefix_ref(xs[0], xs[1], xs[2], eps)
    (out * go.float()).sum().backward()
    return [orc.relerr(x.grad, r) for x, r in zip(xs, ref)]
