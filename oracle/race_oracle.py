"""fp64 CPU restatement of causal RACE attention -- TEST INFRASTRUCTURE ONLY.

This module is the parity oracle. Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker: nothing in ``race_attention_amd`` imports or calls it, and the HIP
product path never falls back to it.

Every function restates the reference's math from the cited file:line in
float64 torch on the CPU (the reference itself is torch code):

  build_planes_protos   scaling/race_common.py:14-33
  soft_hash_probs       scaling/race_common.py:36-73   (softmax form)
  soft_hash_sigmoid     closed form of the same map (product of per-bit
                        sigmoids; independent formula used as a cross-check)
  race_prefix_ref       scaling/race_common.py:76-90   (materialised cumsum)
  race_prefix_brute     O(T^2) double loop of the same definition, tiny T only
  race_module_ref       scaling/race_causal_cuda.py:94-102 / race_torch_cumsum.py:27-36
  decode_ref            state semantics of race_prefix_ref's (A_final, B_final)
                        (the reference has no decode: chat/nanochat/gpt.py:143-146)
  race_noncausal_ref    scaling/benchmark_time.py:139-160 (non-causal bmm sequence)
  race_noncausal_brute  O(T^2) loop of the same definition, tiny T only
  batched_ace_nc_ref    scaling/benchmark_time.py:111-166 (BatchedACE.forward with
                        the learnable temperature, shared or per-ensemble planes)
  causal_linear_ref     kernels/cpu/linear_pref.cpp:87-130 (causal_dot_product), as
                        kernels/cpu/test_cpu_kernels.py:94-97 states it
  causal_linear_brute   O(L^2) loop of out_l = sum_{s<=l} (Q_l . K_s) V_s

How each is pinned (tests/test_oracle.py):
  build_planes_protos : committed fixture of the planes for the seeds used;
                        corners against binary counting.
  soft_hash_probs     : equals soft_hash_sigmoid (two formulas); planes=0 gives
                        exactly 1/R; K=1 gives [sigma(-2u), sigma(2u)]; rows sum
                        to 1; golden vectors written by the reference itself.
  race_prefix_ref     : equals race_prefix_brute; planes=0 known answer
                        out_t = L * sum_{tau<=t} v_tau / (t+1+R*eps); T=1 closed
                        form; equals the C restatement of race_pref.cpp and the
                        compiled reference kernel (oracle/_ref) where built.
  gradients           : torch.autograd of these fp64 functions, pinned by
                        torch.autograd.gradcheck (finite differences) and by the
                        C restatement of the explicit backward in race_pref.cpp.
  decode_ref          : equals race_module_ref at every position.
  race_noncausal_ref  : equals race_noncausal_brute; its last row equals
                        race_prefix_ref's last row (the causal prefix at T-1 is the
                        whole sequence); planes=0 known answer
                        out_t = L * sum_tau v_tau / (T + R*eps); gradients by
                        torch.autograd.gradcheck.
  causal_linear_ref   : equals causal_linear_brute and the compiled reference
                        linear_pref.cpp (oracle/_ref) where built; gradients by
                        gradcheck and against the reference's causal_dot_backward.
  batched_ace_nc_ref  : built from soft_hash_probs' formula with a tensor scale;
                        pinned through race_noncausal_ref and by gradcheck in the
                        temperature.
"""
import itertools
import math

import torch

F64 = torch.float64


def build_planes_protos(d_k, Kbits, L, M=1, share_planes=True, seed=0, dtype=torch.float32):
    """Hyperplanes and corner prototypes (scaling/race_common.py:14-33).

    planes ~ randn(L, Kbits, d_k) from a CPU Generator seeded with ``seed``;
    planes_T = planes.view(L*Kbits, d_k).T -> [d_k, L*Kbits] (column j = l*K + k).
    share_planes=False draws [M, L, Kbits, d_k] -> [M, d_k, L*Kbits].
    protos_T [Kbits, R]: column r is the r-th element of itertools.product([-1,1], repeat=K).
    """
    g = torch.Generator(device="cpu").manual_seed(seed)
    if share_planes:
        planes = torch.randn(L, Kbits, d_k, generator=g)
        planes_T = planes.reshape(L * Kbits, d_k).t().contiguous()
    else:
        planes = torch.randn(M, L, Kbits, d_k, generator=g)
        planes_T = planes.reshape(M, L * Kbits, d_k).transpose(1, 2).contiguous()
    corners = torch.tensor(list(itertools.product([-1.0, 1.0], repeat=Kbits)))
    protos_T = corners.t().contiguous()
    return planes_T.to(dtype), protos_T.to(dtype)


def _pack(X, M):
    """[B,H,T,D] -> [N,T,D] with N ordered (M,B,H) (race_common.py:49-53)."""
    B, H, T, D = X.shape
    return X.unsqueeze(0).expand(M, B, H, T, D).reshape(M * B * H, T, D)


def _proj(X, planes_T, M, share_planes):
    """x @ planes_T per ensemble member (race_common.py:54-63), fp64."""
    B, H, T, D = X.shape
    Xm = _pack(X.to(F64), M)
    P = planes_T.to(F64)
    if share_planes:
        return Xm @ P
    N = M * B * H
    LK = P.shape[-1]
    Pe = P.unsqueeze(1).unsqueeze(1).expand(M, B, H, D, LK).reshape(N, D, LK)
    return torch.bmm(Xm, Pe)


def soft_hash_probs(Q, K, V, planes_T, protos_T, L, Kbits, M=1, share_planes=True, scale=None):
    """Soft bucket probabilities, softmax form (scaling/race_common.py:36-73), in fp64.

    logits[n,t,l,r] = sum_k tanh(proj[n,t,l*K+k]) / scale * protos_T[k,r];
    probs = softmax_r(logits), reshaped to [N,T,L*R] (L-outer, R-inner).
    ``scale`` defaults to sqrt(D) exactly as race_common.py:46.
    Returns (probsK, probsQ, V2, N) with V2 = packed V in fp64.
    """
    B, H, T, D = Q.shape
    R = protos_T.shape[1]
    if scale is None:
        scale = math.sqrt(D)
    N = M * B * H
    pr = protos_T.to(F64)

    def probs(X):
        proj = _proj(X, planes_T, M, share_planes).view(N, T, L, Kbits)
        logits = (proj.tanh() / scale) @ pr
        return torch.softmax(logits, dim=-1).reshape(N, T, L * R)

    return probs(K), probs(Q), _pack(V.to(F64), M), N


def soft_hash_sigmoid(X, planes_T, L, Kbits, M=1, share_planes=True, scale=None):
    """Closed form of the soft-hash: p_l[r] = prod_k sigmoid(2 c_k(r) u_{l,k}).

    With u = tanh(proj)/scale and c(r) the corner of r (bit K-1-k of r set <=> c_k=+1,
    the ordering of itertools.product in race_common.py:30-32), the softmax over the
    2^K corners of sum_k c_k u_k factorises because
    sum_c exp(sum_k c_k u_k) = prod_k (e^{u_k} + e^{-u_k}).
    """
    B, H, T, D = X.shape
    if scale is None:
        scale = math.sqrt(D)
    N = M * B * H
    u = _proj(X, planes_T, M, share_planes).view(N, T, L, Kbits).tanh() / scale
    R = 1 << Kbits
    out = torch.ones(N, T, L, R, dtype=F64)
    for r in range(R):
        for k in range(Kbits):
            c = 1.0 if (r >> (Kbits - 1 - k)) & 1 else -1.0
            out[..., r] = out[..., r] * torch.sigmoid(2.0 * c * u[..., k])
    return out.reshape(N, T, L * R)


def race_prefix_ref(probsK, probsQ, V2, eps=1e-6):
    """Materialised causal prefix scan (scaling/race_common.py:76-90).

    A = cumsum_t pK; B = cumsum_t pK (x) v; out = sum_s pQ * B / (A + eps).
    Returns (out [N,T,D], A_final [N,S], B_final [N,S,D]) in the input dtype.
    """
    A_pref = probsK.cumsum(dim=1)
    B_pref = (probsK.unsqueeze(-1) * V2.unsqueeze(2)).cumsum(dim=1)
    E_pref = B_pref / (A_pref.unsqueeze(-1) + eps)
    out = torch.einsum("nts,ntsd->ntd", probsQ, E_pref)
    return out, A_pref[:, -1].contiguous(), B_pref[:, -1].contiguous()


def race_prefix_brute(probsK, probsQ, V2, eps=1e-6):
    """Definition of the causal RACE readout as explicit loops (tiny inputs only).

    out[n,t,:] = sum_s pQ[n,t,s] * (sum_{tau<=t} pK[n,tau,s] v[n,tau,:]) /
                 (sum_{tau<=t} pK[n,tau,s] + eps)
    (forward_kernel.cu:4-6, race_pref.cpp:23-27).
    """
    N, T, S = probsK.shape
    D = V2.shape[2]
    out = torch.zeros(N, T, D, dtype=F64)
    for n in range(N):
        for t in range(T):
            acc = torch.zeros(D, dtype=F64)
            for s in range(S):
                a = 0.0
                b = torch.zeros(D, dtype=F64)
                for tau in range(t + 1):
                    w = float(probsK[n, tau, s])
                    a += w
                    b += w * V2[n, tau].to(F64)
                acc += float(probsQ[n, t, s]) * b / (a + eps)
            out[n, t] = acc
    return out


def race_module_ref(Q, K, V, planes_T, protos_T, L, Kbits, M=1, share_planes=True,
                    eps=1e-6, scale=None):
    """Module forward [B,H,T,D] -> [B,H,T,D] (race_causal_cuda.py:94-102 and
    race_torch_cumsum.py:27-36): soft-hash, prefix scan, mean over the M ensemble
    copies. fp64 and differentiable w.r.t. Q, K, V."""
    B, H, T, D = Q.shape
    pK, pQ, V2, N = soft_hash_probs(Q, K, V, planes_T, protos_T, L, Kbits, M, share_planes, scale)
    out, _, _ = race_prefix_ref(pK, pQ, V2, eps)
    return out.view(M, B, H, T, D).mean(dim=0)


def race_gqa_ref(Q, K, V, planes_T, L, Kbits, eps=1e-6, scale=None):
    """Grouped-query RACE: Q [B,Hq,T,D], K/V [B,Hkv,T,D]; query head h reads the
    bucket state of kv head h // (Hq/Hkv). Defined as MHA with K,V repeated over
    the group (the reference asserts Hq == Hkv, chat/nanochat/gpt.py:96)."""
    Hq, Hkv = Q.shape[1], K.shape[1]
    rep = Hq // Hkv
    Kr = K.repeat_interleave(rep, dim=1)
    Vr = V.repeat_interleave(rep, dim=1)
    _, protos_T = build_planes_protos(Q.shape[-1], Kbits, L)
    return race_module_ref(Q, Kr, Vr, planes_T, protos_T, L, Kbits, 1, True, eps, scale)


def decode_ref(K_hist, V_hist, q_new, k_new, v_new, planes_T, L, Kbits, eps=1e-6, scale=None):
    """One decode step from scratch: the state after the prefix (A_final, B_final of
    race_prefix_ref over K_hist/V_hist plus the new token), read out by q_new.

    K_hist, V_hist [B,H,T,D]; q_new/k_new/v_new [B,H,D]. Returns (out [B,H,D],
    A [B*H,S], Bst [B*H,S,D]) -- the out row equals race_module_ref at position T.
    """
    _, protos_T = build_planes_protos(q_new.shape[-1], Kbits, L)
    Kf = torch.cat([K_hist, k_new.unsqueeze(2)], dim=2)
    Vf = torch.cat([V_hist, v_new.unsqueeze(2)], dim=2)
    Qf = torch.cat([torch.zeros_like(K_hist), q_new.unsqueeze(2)], dim=2)
    pK, pQ, V2, N = soft_hash_probs(Qf, Kf, Vf, planes_T, protos_T, L, Kbits, 1, True, scale)
    out, A, Bst = race_prefix_ref(pK, pQ, V2, eps)
    Bb, H = q_new.shape[0], q_new.shape[1]
    return out[:, -1].reshape(Bb, H, -1), A, Bst


def race_noncausal_ref(probsK, probsQ, V2, eps=1e-6):
    """Non-causal bucket summaries (scaling/benchmark_time.py:139-160):
    A = sum_t pK, B = pK^T V, E = B / (A + eps), out = pQ E. [N,T,S] x2, [N,T,D] -> [N,T,D]."""
    A = probsK.sum(dim=1)
    Bsum = probsK.transpose(1, 2) @ V2
    E = Bsum / (A.unsqueeze(-1) + eps)
    return probsQ @ E


def race_noncausal_brute(probsK, probsQ, V2, eps=1e-6):
    """O(N T^2 S) loops of out[t] = sum_s pQ[t,s] sum_tau pK[tau,s] v_tau / (sum_tau pK[tau,s] + eps)."""
    N, T, S = probsK.shape
    out = torch.zeros(N, T, V2.shape[-1], dtype=F64)
    for n in range(N):
        for s in range(S):
            a = float(probsK[n, :, s].sum())
            b = (probsK[n, :, s].to(F64).unsqueeze(-1) * V2[n].to(F64)).sum(0)
            for t in range(T):
                out[n, t] += float(probsQ[n, t, s]) * b / (a + eps)
    return out


def batched_ace_nc_ref(Khf, Vhf, Qhf, planes_T, protos_T, L, Kbits, share_planes, logit_temp, eps=1e-6,
                       dtype=F64):
    """BatchedACE.forward of scaling/benchmark_time.py:111-166 in fp64 (or, as bench.py's CPU
    baseline, in the reference's own fp32 with dtype=torch.float32).

    Khf, Vhf, Qhf [M,B,T,H,dk]; planes_T [dk, L*K] (shared) or [M, dk, L*K];
    logit_temp a 0-d tensor: scale = exp(logit_temp).clamp(1e-2, 10) divides the
    tanh'd projections. Differentiable in the inputs and logit_temp."""
    M, B, T, H, dk = Khf.shape
    N = M * B * H
    S = L << Kbits
    scale = logit_temp.to(dtype).exp().clamp(1e-2, 10.0)

    def flat(X):
        return X.to(dtype).permute(0, 1, 3, 2, 4).reshape(M, B * H, T, dk)

    Kh, Qh, Vh = flat(Khf), flat(Qhf), flat(Vhf)
    P = planes_T.to(dtype)
    pr = protos_T.to(dtype)

    def probs(Xh):
        proj = Xh @ P if share_planes else torch.einsum("mbtd,mds->mbts", Xh, P)
        logits = (proj.reshape(N, T, L, Kbits).tanh() / scale) @ pr
        return torch.softmax(logits, dim=-1).reshape(N, T, S)

    out = race_noncausal_ref(probs(Kh), probs(Qh), Vh.reshape(N, T, dk), eps)
    return out.view(M, B, H, T, dk).permute(0, 1, 3, 2, 4)


def causal_linear_ref(Q, K, V):
    """Causal linear attention (kernels/cpu/linear_pref.cpp:87-130): out_l = Q_l .
    sum_{s<=l} K_s (x) V_s. Q, K [N,H,L,E], V [N,H,L,M] -> [N,H,L,M], fp64."""
    KV = (K.to(F64).unsqueeze(-1) * V.to(F64).unsqueeze(-2)).cumsum(2)
    return (Q.to(F64).unsqueeze(-1) * KV).sum(-2)


def causal_linear_brute(Q, K, V):
    N, H, L, _ = Q.shape
    out = torch.zeros(N, H, L, V.shape[-1], dtype=F64)
    for l in range(L):
        for s in range(l + 1):
            out[:, :, l] += (Q[:, :, l].to(F64) * K[:, :, s].to(F64)).sum(-1, keepdim=True) * V[:, :, s].to(F64)
    return out


def relerr(got, ref):
    """max|got-ref| / max|ref| -- the reference's error metric
    (scaling/test_kernels.py:30-31)."""
    g = got.detach().to(F64).cpu()
    r = ref.detach().to(F64).cpu()
    return (g - r).abs().max().item() / (r.abs().max().item() + 1e-30)


def maxabs(got, ref):
    return (got.detach().to(F64).cpu() - ref.detach().to(F64).cpu()).abs().max().item()
