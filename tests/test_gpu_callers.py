"""The reference's callers on the GPU: misc/race.py's RACEAttention / RACEBlock and the nanochat
attention seam (chat/nanochat/gpt.py:109-151), each against an fp64 restatement of the caller
built on the pinned oracle."""
import math

import pytest
import torch

from oracle import race_oracle as orc
from race_ref import bf16_planes, check

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _attention_ref(att, x, merge):
    """fp64 RACEAttention.forward (misc/race.py:160-173) with the module's own weights: q/k/v
    projections, per-head causal RACE (oracle), the ensemble mean (shared planes: one copy) and
    the chosen head merge, then the output projection."""
    B, T, d = x.shape
    h, dk = att.h, att.d_k
    W = {n: (getattr(att, n).weight.detach().double().cpu(),
             None if getattr(att, n).bias is None else getattr(att, n).bias.detach().double().cpu())
         for n in ("q", "k", "v", "o")}
    x64 = x.detach().double().cpu()

    def lin(n, z):
        w, b = W[n]
        return z @ w.T + (0 if b is None else b)

    Q, K, V = (lin(n, x64).view(B, T, h, dk).transpose(1, 2) for n in ("q", "k", "v"))
    planes = att.ace.planes_T.detach().double().cpu()
    _, protos = orc.build_planes_protos(dk, att.ace.K, att.ace.L)
    out = orc.race_module_ref(Q, K, V, planes, protos, att.ace.L, att.ace.K, eps=EPS)  # [B,H,T,dk]
    if merge == "reference":
        y = out.contiguous().view(B, T, -1)  # [B,H,T,dk] memory read as [B,T,H*dk] (misc/race.py:171)
    else:
        y = out.transpose(1, 2).contiguous().view(B, T, -1)
    return lin("o", y)


@pytest.mark.parametrize("merge", ["reference", "heads"])
@pytest.mark.parametrize("M", [1, 3])
def test_race_attention_matches_fp64(dev, merge, M):
    """RACEAttention (fp32 activations: HIP soft-hash + fp32 scan) at the 1e-4 fp32 bar, with the
    reference's head merge (which mixes heads and tokens) and with the per-token merge."""
    from race_attention_amd import RACEAttention
    torch.manual_seed(3)
    att = RACEAttention(128, 4, 3, 4, M, drop=0.0, device=dev, merge=merge).to(dev).eval()
    x = torch.randn(2, 150, 128, device=dev)
    y = att(x)
    check(f"RACEAttention merge={merge} M={M}", y, _attention_ref(att, x, merge), 1e-4)


def test_race_attention_reference_merge_is_not_causal(dev):
    """The reference merge reads later tokens (misc/race.py:171): changing the last token changes
    the first output rows; the per-token merge keeps them causal."""
    from race_attention_amd import RACEAttention
    torch.manual_seed(4)
    x = torch.randn(1, 64, 128, device=dev)
    x2 = x.clone()
    x2[:, -1] += 1.0
    for merge, causal in (("reference", False), ("heads", True)):
        att = RACEAttention(128, 4, 3, 4, 1, drop=0.0, device=dev, merge=merge).to(dev).eval()
        with torch.no_grad():
            same = torch.equal(att(x)[:, :-1], att(x2)[:, :-1])
        assert same == causal, merge


def test_race_block_matches_fp64_and_trains(dev):
    """RACEBlock (misc/race.py:176-206): pre-norm attention + MLP residuals against fp64 with the
    block's own weights, and a backward pass reaching every parameter."""
    from race_attention_amd import RACEBlock
    torch.manual_seed(5)
    cfg = {"emb_dim": 128, "n_heads": 2, "K": 4, "L": 8, "M": 1, "drop_rate": 0.0, "qkv_bias": True}
    blk = RACEBlock(cfg, device=dev).to(dev).eval()
    x = torch.randn(2, 100, 128, device=dev, requires_grad=True)
    y = blk(x)
    ln1 = torch.nn.functional.layer_norm
    x64 = x.detach().double().cpu()
    n1 = ln1(x64, (128,), blk.norm1.weight.detach().double().cpu(), blk.norm1.bias.detach().double().cpu())
    h1 = x64 + _attention_ref(blk.att, n1, "reference")
    n2 = ln1(h1, (128,), blk.norm2.weight.detach().double().cpu(), blk.norm2.bias.detach().double().cpu())
    ff = [m for m in blk.ff if isinstance(m, torch.nn.Linear)]
    a = n2 @ ff[0].weight.detach().double().cpu().T + ff[0].bias.detach().double().cpu()
    a = torch.nn.functional.gelu(a)
    ref = h1 + a @ ff[1].weight.detach().double().cpu().T + ff[1].bias.detach().double().cpu()
    check("RACEBlock", y, ref, 1e-4)
    y.square().mean().backward()
    assert all(p.grad is not None and torch.isfinite(p.grad).all() for p in blk.parameters() if p.requires_grad)


def _seam_qkv(dev, n_head, n_kv_head, T, seed):
    from race_attention_amd.nanochat import CausalSelfAttention, GPTConfig, apply_rotary_emb, norm, rotary_tables
    cfg = GPTConfig(n_layer=1, n_head=n_head, n_kv_head=n_kv_head, n_embd=64 * n_head, race_l=8, race_k=4)
    torch.manual_seed(seed)
    attn = CausalSelfAttention(cfg, 0).to(dev)
    attn.init_race_buffers()
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(1, T, cfg.n_embd, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    cos, sin = rotary_tables(T, 64, device=dev)
    with torch.no_grad():
        q = attn.c_q(x).view(1, T, n_head, 64)
        k = attn.c_k(x).view(1, T, n_kv_head, 64)
        v = attn.c_v(x).view(1, T, n_kv_head, 64)
        q, k = norm(apply_rotary_emb(q, cos, sin)) * 1.2, norm(apply_rotary_emb(k, cos, sin)) * 1.2
    return cfg, attn, q, k, v


@pytest.mark.parametrize("n_head,n_kv_head", [(4, 4), (4, 2)])
def test_seam_fp32_matches_reference_semantics(dev, n_head, n_kv_head):
    """The seam's default precision is gpt.py:132-140: fp32 q/k/v, fp32 planes, fp32 scan. Its
    attention core equals the fp64 oracle with the planes at full precision (the fused path would
    round them to bf16); the bf16 output is the only rounding, hence the bf16 bar."""
    from race_attention_amd.nanochat import race_attend
    cfg, attn, q, k, v = _seam_qkv(dev, n_head, n_kv_head, 300, seed=6)
    with torch.no_grad():
        y = race_attend(q, k, v, attn.planes_T, cfg.race_l, cfg.race_k, cfg.race_eps, precision="fp32",
                        protos_T=attn.protos_T)
    pl = attn.planes_T.detach().double().cpu()
    ref = orc.race_gqa_ref(q.transpose(1, 2).double().cpu(), k.transpose(1, 2).double().cpu(),
                           v.transpose(1, 2).double().cpu(), pl, cfg.race_l, cfg.race_k, cfg.race_eps)
    assert y.dtype == q.dtype
    re = check("seam fp32", y.transpose(1, 2), ref, 2e-2)
    # before the cast to the activation dtype it is the fp32 path at the fp32 bar
    from race_attention_amd.nanochat import race_attend_fp32
    qf, kf, vf = q.float(), k.float(), v.float()
    y32 = race_attend_fp32(qf, kf, vf, attn.planes_T, attn.protos_T, cfg.race_l, cfg.race_k, cfg.race_eps)
    re32 = check("seam fp32 before the cast", y32.transpose(1, 2), ref, 1e-4)
    print(f"seam fp32 relerr {re:.2e} (bf16 output), {re32:.2e} (fp32)")


def test_seam_bf16_matches_bf16_planes_oracle(dev):
    """race_precision="bf16": the fused kernels, pinned against the fp64 oracle with the planes
    rounded to bf16 (what the fused kernels use) and, at the same bar, with fp32 planes."""
    from race_attention_amd.nanochat import race_attend
    cfg, attn, q, k, v = _seam_qkv(dev, 4, 2, 300, seed=7)
    with torch.no_grad():
        y = race_attend(q, k, v, attn.planes_T, cfg.race_l, cfg.race_k, cfg.race_eps, precision="bf16")
    args = (q.transpose(1, 2).double().cpu(), k.transpose(1, 2).double().cpu(), v.transpose(1, 2).double().cpu())
    for name, pl in (("bf16 planes", bf16_planes(attn.planes_T)), ("fp32 planes", attn.planes_T)):
        ref = orc.race_gqa_ref(*args, pl.detach().double().cpu(), cfg.race_l, cfg.race_k, cfg.race_eps)
        print(f"seam bf16 vs oracle with {name}: relerr {check('seam bf16 ' + name, y.transpose(1, 2), ref, 2e-2):.2e}")


def test_seam_module_default_runs_fp32_path(dev):
    """CausalSelfAttention with the default config runs the fp32 path forward and backward
    (the reference seam's gradients flow through the HIP soft-hash and op kernels)."""
    from race_attention_amd.nanochat import CausalSelfAttention, GPTConfig, rotary_tables
    cfg = GPTConfig(n_layer=2, n_head=2, n_kv_head=2, n_embd=128, race_l=3, race_k=3)
    attn = CausalSelfAttention(cfg, 1).to(dev)
    attn.init_race_buffers()
    x = torch.randn(2, 40, 128, device=dev, dtype=torch.bfloat16, requires_grad=True)
    ve = torch.randn(2, 40, 128, device=dev, dtype=torch.bfloat16)
    cos, sin = rotary_tables(40, 64, device=dev)
    y = attn(x, ve, (cos, sin), None, None)
    y.float().square().mean().backward()
    assert y.dtype == torch.bfloat16 and torch.isfinite(x.grad.float()).all()
