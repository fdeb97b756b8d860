"""BASELINE.json configurations on the GPU, at their full sizes.

cfg1 (the reference's CPU plumbing case, fp32) is checked whole against the fp64 oracle,
outputs and gradients, at both the reference's scale sqrt(D) and the literal temperature 1.0.

cfg2 (T = 65536, S = 256: two bucket tiles whose partial outputs are summed) and cfg3
(T = 2^20) run forward and backward at their full size; out, dq, dk and dv are compared with
the fp64 oracle on token windows of whole streams: the first tokens, windows straddling the
workgroup block boundaries (first, middle and last: the carried block states and, for the
backward, the suffix states of every later block) and the sequence end. The oracle scans each
checked stream completely (oracle_c.race_windows), so every window sees its exact prefix and,
backward, its exact suffix. Each window is normalised by itself (reference pass rule,
scaling/test_kernels.py:38-51, per window), so late windows, whose gradients are orders of
magnitude smaller than the first tokens', are held to the same relative bar.

The long-context sweep (T = 2^21 .. 2^24) runs forward and backward at full size; out, dq, dk
and dv are checked on windows across the last block boundary and at the sequence end (the oracle
starts from the fp64 prefix state of everything before them and scans to the end), and out and dq
across the middle block boundary (dk and dv there too at T = 2^22, over the whole suffix).
"""
import math

import pytest
import torch

from race_ref import (bf16_planes, check, oracle_group_windows, oracle_layer, oracle_prefix_state,
                      oracle_segment_windows, qkv_blocks)

pytestmark = pytest.mark.gpu

EPS = 1e-6
BF16_TOL = 2e-2
FP32_TOL = 1e-4


@pytest.mark.parametrize("scale", [None, 1.0])
def test_cfg1_fp32_layer(dev, scale):
    """B=2, H=8, T=2048, D=64, L=8, K=4, fp32, q/k/v ~ N(0,1), upstream grad ~ N(0,1):
    outputs and gradients within the north star's fp32 bar 1e-4."""
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
    for name, got, r in (("out", out, ref), ("dq", q.grad, dq), ("dk", k.grad, dk), ("dv", v.grad, dv)):
        print(f"cfg1 scale={s} {name} relerr {check('cfg1 ' + name, got, r, FP32_TOL):.2e}")


def _inputs(dev, B, Hq, Hkv, T, D, std, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    q = (torch.randn(B, Hq, T, D, generator=g, device=dev) * std).to(torch.bfloat16)
    k = (torch.randn(B, Hkv, T, D, generator=g, device=dev) * std).to(torch.bfloat16)
    v = (torch.randn(B, Hkv, T, D, generator=g, device=dev) * std).to(torch.bfloat16)
    go = torch.randn(B, Hq, T, D, generator=g, device=dev).to(torch.bfloat16)
    return q, k, v, go


def _boundary_windows(T, CB, NB, wlen):
    """Window starts: the first tokens, across the first, a middle and the last block boundary,
    and the sequence end."""
    wins = {0, T - wlen}
    for b in sorted({1, NB // 2, NB - 1}):
        if 0 < b < NB:
            wins.add(min(max(b * CB - wlen // 2, 0), T - wlen))
    wins = sorted(wins)
    out = []
    for w in wins:  # disjoint
        if not out or w >= out[-1] + wlen:
            out.append(w)
    return out


def _check_windows(tag, got, ref, wins, wlen, tol):
    """got [nwin*, wlen, D] rows of the GPU result (any dtype), ref fp64: each window on its own."""
    for i, w in enumerate(wins):
        re = check(f"{tag} window [{w}, {w + wlen})", got[i], ref[i], tol)
        print(f"{tag} window [{w},{w + wlen}) relerr {re:.2e}", flush=True)


def _full_size(dev, B, Hq, Hkv, T, D, L, Kb, std, seed, streams, wlen=128):
    from race_attention_amd import build_planes_protos, race_causal_attention
    print(f"full-size B={B} H={Hq}/{Hkv} T={T} D={D} L={L} K={Kb}", flush=True)
    planes_T, _ = build_planes_protos(D, Kb, L, 1, device=dev, seed=0)
    q, k, v, go = _inputs(dev, B, Hq, Hkv, T, D, std, seed)
    xs = [x.clone().requires_grad_(True) for x in (q, k, v)]
    out = race_causal_attention(*xs, planes_T, L, Kb, eps=EPS)
    out.backward(go)
    grads = [x.grad for x in xs]
    for x in grads:
        assert torch.isfinite(x.float()).all()
    CB, NB = qkv_blocks(T, B * Hkv, L, Kb, D)
    wins = _boundary_windows(T, CB, NB, wlen)
    print(f"block {CB} tokens x {NB} blocks; windows {wins}", flush=True)
    idx = torch.cat([torch.arange(w, w + wlen) for w in wins]).to(dev)
    pl = bf16_planes(planes_T)
    G = Hq // Hkv
    for (b, hk) in streams:
        r_out, r_dq, r_dk, r_dv = oracle_group_windows(q, k, v, go, pl, L, Kb, math.sqrt(D), EPS, b, hk, wins, wlen)
        nw = len(wins)
        for gi in range(G):
            h = hk * G + gi
            _check_windows(f"b{b} h{h} out", out[b, h, idx].view(nw, wlen, D), r_out[gi], wins, wlen, BF16_TOL)
            _check_windows(f"b{b} h{h} dq", grads[0][b, h, idx].view(nw, wlen, D), r_dq[gi], wins, wlen, BF16_TOL)
        _check_windows(f"b{b} kv{hk} dk", grads[1][b, hk, idx].view(nw, wlen, D), r_dk, wins, wlen, BF16_TOL)
        _check_windows(f"b{b} kv{hk} dv", grads[2][b, hk, idx].view(nw, wlen, D), r_dv, wins, wlen, BF16_TOL)
    # bitwise determinism of the full-size backward
    ys = [x.detach().clone().requires_grad_(True) for x in (q, k, v)]
    race_causal_attention(*ys, planes_T, L, Kb, eps=EPS).backward(go)
    for a, y in zip(grads, ys):
        assert torch.equal(a, y.grad), "full-size backward is not deterministic"


def test_cfg2_full_size(dev):
    """B=4, H=16, T=65536, D=64, L=16, K=4 (S=256: two bucket tiles and their partial sums),
    bf16 ~ N(0,1): streams (0, 0) and (3, 15) on windows across every kind of block boundary."""
    _full_size(dev, 4, 16, 16, 65536, 64, 16, 4, 1.0, seed=2, streams=[(0, 0), (3, 15)])


def test_cfg3_full_size(dev):
    """B=1, H=4, T=2^20, D=64, L=8, K=4, bf16 ~ N(0, 1/sqrt(D)): heads 0 and 3 on windows at
    the start, across the first, middle and last of the ~192 block boundaries, and at the end."""
    _full_size(dev, 1, 4, 4, 1 << 20, 64, 8, 4, 1.0 / math.sqrt(64), seed=1, streams=[(0, 0), (0, 3)])


def test_gqa_long_full_size(dev):
    """Grouped-query heads over a long sequence (B=1, 8 query / 2 kv heads, T=2^18): the
    query-head loop inside the fused kernels across block boundaries, dk/dv summed over groups."""
    _full_size(dev, 1, 8, 2, 1 << 18, 64, 8, 4, 1.0 / math.sqrt(64), seed=5, streams=[(0, 1)])


def test_fused_t65536_whole(dev):
    """The fused layer at T = 65536 with the automatic block count, every token of every output
    and gradient against the fp64 oracle (the fused tests elsewhere stop at T = 4096)."""
    from race_attention_amd import build_planes_protos, race_causal_attention
    B, H, T, D, L, Kb = 1, 2, 65536, 64, 8, 4
    planes_T, _ = build_planes_protos(D, Kb, L, 1, device=dev, seed=0)
    q, k, v, go = _inputs(dev, B, H, H, T, D, 1.0 / math.sqrt(D), seed=9)
    xs = [x.clone().requires_grad_(True) for x in (q, k, v)]
    out = race_causal_attention(*xs, planes_T, L, Kb, eps=EPS)
    out.backward(go)
    ref = oracle_layer(q, k, v, bf16_planes(planes_T), L, Kb, math.sqrt(D), EPS, go)
    for name, got, r in zip(("out", "dq", "dk", "dv"), [out] + [x.grad for x in xs], ref):
        print(f"T=65536 whole {name} relerr {check(name, got, r, BF16_TOL):.2e}", flush=True)


@pytest.mark.parametrize("T", [1 << 21, 1 << 22, 1 << 23, 1 << 24])
def test_cfg3_sweep_fwd_bwd(dev, T):
    """The long-context sweep (B=1, H=4, D=64, L=8, K=4, bf16 ~ N(0, 1/sqrt(D)), go ~ N(0,1)) at
    every T it runs, forward and backward at full size, against the fp64 oracle
    (scaling/test_kernels.py:69-104 checks gradients at every T of its sweep):
      * the tail: out, dq, dk, dv of head 2 on a window across the last workgroup-block boundary
        and on the sequence's last tokens; the oracle starts from the exact fp64 prefix state of
        every earlier token and scans the tail to the end, so the suffix sums are exact;
      * the middle: out and dq (which depend only on the prefix) on a window across the middle
        block boundary; at T = 2^22 also dk and dv there, with the oracle scanning the whole
        2M-token suffix."""
    from race_attention_amd import build_planes_protos, race_causal_attention
    B, H, D, L, Kb, wlen, h = 1, 4, 64, 8, 4, 256, 2
    print(f"cfg3 sweep T={T} fwd+bwd", flush=True)
    planes_T, _ = build_planes_protos(D, Kb, L, 1, device=dev, seed=0)
    q, k, v, go = _inputs(dev, B, H, H, T, D, 1.0 / math.sqrt(D), seed=1)
    xs = [x.requires_grad_(True) for x in (q, k, v)]
    out = race_causal_attention(*xs, planes_T, L, Kb, eps=EPS)
    out.backward(go)
    torch.cuda.synchronize()
    grads = [x.grad for x in xs]
    for x in grads:
        assert torch.isfinite(x.float()).all()
    q, k, v = (x.detach() for x in xs)
    CB, NB = qkv_blocks(T, B * H, L, Kb, D)
    pl = bf16_planes(planes_T)
    scale = math.sqrt(D)
    names = ("out", "dq", "dk", "dv")
    got_all = [out] + grads

    def compare(tag, wins, refs, which):
        idx = torch.cat([torch.arange(w, w + wlen) for w in wins]).to(dev)
        for name, got, ref in zip(names, got_all, refs):
            if name in which:
                _check_windows(f"T={T} {tag} h{h} {name}", got[0, h, idx].view(len(wins), wlen, D), ref, wins, wlen,
                               BF16_TOL)

    # tail: from just before the last block boundary to the end
    last = (NB - 1) * CB
    t0 = max(last - wlen, 0)
    wins = sorted({min(max(last - wlen // 2, t0), T - 2 * wlen), T - wlen})
    print(f"block {CB} tokens x {NB} blocks; tail [{t0}, {T}) windows {wins}", flush=True)
    refs = oracle_segment_windows(q, k, v, go, pl, L, Kb, scale, EPS, 0, h, t0, T, wins, wlen)
    compare("tail", wins, refs, names)
    # middle block boundary
    mid = (NB // 2) * CB - wlen // 2
    if T == 1 << 22:
        refs = oracle_segment_windows(q, k, v, go, pl, L, Kb, scale, EPS, 0, h, mid, T, [mid], wlen)
        compare("middle (full suffix)", [mid], refs, names)
    else:
        refs = oracle_segment_windows(q, k, v, go, pl, L, Kb, scale, EPS, 0, h, mid, mid + wlen, [mid], wlen)
        compare("middle", [mid], refs, ("out", "dq"))


def test_cfg4_decode_at_baseline_shape(dev):
    """cfg4: 256 sequences, 32 query / 8 kv heads, D=64, L=8, K=4, a 512-token prefill by the
    fused forward, then 1024 single-token decode steps on the carried fp32 state. Outputs of the
    first, middle and last 16 steps and the final (A, Bs) state of three (sequence, kv head)
    pairs against the fp64 oracle of the whole 1536-token sequence."""
    from race_attention_amd import RaceDecodeState, build_planes_protos
    B, Hq, Hkv, D, L, Kb, T0, steps = 256, 32, 8, 64, 8, 4, 512, 1024
    T = T0 + steps
    planes_T, _ = build_planes_protos(D, Kb, L, 1, device=dev, seed=0)
    g = torch.Generator(device=dev).manual_seed(1)
    q = torch.randn(B, Hq, T, D, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, Hkv, T, D, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B, Hkv, T, D, generator=g, device=dev).to(torch.bfloat16)
    st = RaceDecodeState(B, Hq, Hkv, D, L, Kb, planes_T, device=dev)
    st.prefill(q[:, :, :T0], k[:, :, :T0], v[:, :, :T0])
    checked = list(range(16)) + list(range(500, 516)) + list(range(steps - 16, steps))
    outs = {}
    for i in range(steps):
        o = st.step(q[:, :, T0 + i].contiguous(), k[:, :, T0 + i].contiguous(), v[:, :, T0 + i].contiguous())
        if i in checked:
            outs[i] = o.clone()
    assert st.tokens == T
    wins, wlen = [T0, T0 + 500, T0 + steps - 16], 16
    pl = bf16_planes(planes_T)
    G = Hq // Hkv
    for (b, hk) in ((0, 0), (77, 3), (255, 7)):
        ref = oracle_group_windows(q, k, v, None, pl, L, Kb, math.sqrt(D), EPS, b, hk, wins, wlen)
        for wi, w in enumerate(wins):
            got = torch.stack([outs[t - T0][b, hk * G:(hk + 1) * G] for t in range(w, w + wlen)], 1)  # [G, wlen, D]
            re = check(f"decode b{b} kv{hk} steps [{w - T0}, {w - T0 + wlen})", got, ref[:, wi], BF16_TOL)
            print(f"cfg4 b{b} kv{hk} decode steps [{w - T0},{w - T0 + wlen}) relerr {re:.2e}", flush=True)
        A_ref, B_ref = oracle_prefix_state(k[b, hk], v[b, hk], pl, L, Kb, math.sqrt(D))
        z = b * Hkv + hk
        ra = check(f"state A b{b} kv{hk}", st.A[z], A_ref, 1e-3)
        rb = check(f"state Bs b{b} kv{hk}", st.Bs[z], B_ref, BF16_TOL)
        print(f"cfg4 b{b} kv{hk} final state relerr A {ra:.2e} Bs {rb:.2e}", flush=True)


def test_cfg5_hybrid_at_baseline_shape(dev):
    """cfg5: the Llama-3.2-1B-shaped hybrid (16 layers, hidden 2048, 32/8 heads of 64, SwiGLU
    8192, RACE L=8 K=4 in every layer), random init, B=8, T=8192 token ids uniform over 128256:
      * the prefill forward+backward gives a finite loss near ln(vocab) and finite gradients;
      * the attention core of one layer at its real q/k/v (G=4 query heads per kv head) matches
        the fp64 oracle on windows across the sequence;
      * a cached prefill plus decode steps equals the full forward at those positions."""
    from race_attention_amd.hybrid import HybridConfig, HybridLM
    from race_attention_amd.nanochat import race_attend
    cfg = HybridConfig()
    torch.manual_seed(0)
    model = HybridLM(cfg).to(dev).init_weights(seed=0)
    B, T = 8, 8192
    g = torch.Generator(device=dev).manual_seed(1)
    idx = torch.randint(0, cfg.vocab_size, (B, T + 4), generator=g, device=dev)
    # one layer's q, k, v as the layer sees them (captured by a forward hook on its attention)
    seen = {}
    layer = model.blocks[5].attn

    def grab(mod, args):
        x, (cos, sin) = args[0], args[1]
        with torch.no_grad():
            Bq, Tq, _ = x.shape
            qq = mod.q_proj(x).view(Bq, Tq, mod.n_head, mod.head_dim)
            kk = mod.k_proj(x).view(Bq, Tq, mod.n_kv_head, mod.head_dim)
            vv = mod.v_proj(x).view(Bq, Tq, mod.n_kv_head, mod.head_dim)
            from race_attention_amd.nanochat import apply_rotary_emb
            seen["qkv"] = (apply_rotary_emb(qq, cos, sin), apply_rotary_emb(kk, cos, sin), vv)

    h = layer.register_forward_pre_hook(grab)
    loss = model(idx[:, :T], targets=idx[:, 1:T + 1])
    h.remove()
    loss.backward()
    print(f"cfg5 prefill loss {loss.item():.4f} (ln vocab {math.log(cfg.vocab_size):.4f})", flush=True)
    assert math.isfinite(loss.item()) and abs(loss.item() - math.log(cfg.vocab_size)) < 1.0
    for n, p in model.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad.float()).all(), n
    model.zero_grad(set_to_none=True)
    qq, kk, vv = seen["qkv"]
    with torch.no_grad():
        y = race_attend(qq, kk, vv, layer.planes_T, cfg.race_l, cfg.race_k, cfg.race_eps)  # [B,T,Hq,D]
    qt, kt, vt, yt = (z.transpose(1, 2) for z in (qq, kk, vv, y))
    wins, wlen = [0, T // 2 - 64, T - 128], 128
    pl = bf16_planes(layer.planes_T)
    for (b, hk) in ((0, 0), (7, 5)):
        ref = oracle_group_windows(qt, kt, vt, None, pl, cfg.race_l, cfg.race_k, math.sqrt(64), cfg.race_eps, b, hk,
                                   wins, wlen)
        for wi, w in enumerate(wins):
            got = yt[b, hk * 4:(hk + 1) * 4, w:w + wlen]
            re = check(f"cfg5 layer 5 b{b} kv{hk} window [{w}, {w + wlen})", got, ref[:, wi], BF16_TOL)
            print(f"cfg5 layer5 b{b} kv{hk} window [{w},{w + wlen}) relerr {re:.2e}", flush=True)
    del seen, qq, kk, vv, y, qt, kt, vt, yt
    # cached prefill of T tokens + 4 decode steps against the full forward of T + 4 tokens
    with torch.no_grad():
        full = model(idx)[:, T - 1:]  # logits at positions T-1 .. T+3
        cache = model.make_cache(B)
        inc = [model(idx[:, :T], cache)[:, -1]]
        for i in range(4):
            inc.append(model(idx[:, T + i:T + i + 1], cache)[:, -1])
    inc = torch.stack(inc, 1)
    err = (inc - full).abs().max().item()
    scale = full.abs().max().item()
    print(f"cfg5 cached prefill+decode vs full forward logits: max abs diff {err:.3e} (max |logit| {scale:.3e})")
    assert err <= BF16_TOL * scale
