"""Hybrid-model seam: the attention layer of chat/nanochat/gpt.py:81-151 on the MI355X kernels.

The reference's CausalSelfAttention (gpt.py:81-151) projects q, k, v, applies the value
embedding gate, rotary embeddings, QK norm and the 1.2 sharpening, then runs RACE through
soft_hash_probs + RaceCausalFn in fp32 (gpt.py:132-140). It asserts n_kv_head == n_head
(gpt.py:97) and raises NotImplementedError for a KV cache (gpt.py:143-146).

This module keeps the same constructor, parameter and buffer names (c_q, c_k, c_v, c_proj,
ve_gate, planes_T [head_dim, L*K], protos_T [K, 2^K]) so checkpoints load with strict=True,
and runs the attention core on the HIP kernels:
  * race_precision "fp32" (the default) is the reference's computation without a cache:
    q, k, v cast to fp32, the soft-hash with fp32 planes (race_soft_hash_fwd) and the fp32
    chunked scan (RaceCausalFn), the output cast back to the activation dtype (gpt.py:132-140);
    any head dim and hash bits the soft-hash covers;
  * race_precision "bf16" runs the fused bf16 kernels (race_qkv_fwd/bwd): planes and bucket
    probabilities rounded to bf16 inside the kernels, bf16 output; head dim 64 or 128, K <= 4;
  * grouped-query attention: query head h reads kv head h // (n_head / n_kv_head) (the fp32
    path repeats k and v over each group, the fused kernels read the shared state);
  * the KV cache is the RACE bucket state (A [S], B [S, D] per kv head), carried by
    RaceStateCache: a prompt is prefilled by the fused forward, which leaves the state,
    and each further token is one race_decode_step kernel. The reference has no cache path
    (gpt.py:143-146), so this one always runs the fused bf16 kernels.
With share_planes=True every ensemble copy of the reference uses the same planes, so its
mean over race_m copies equals one copy (race_common.py:49-57); race_m is kept as a field.
"""
import math
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from .attention import race_causal_attention
from .decode import RaceDecodeState
from .race_causal_cuda import RaceCausalFn
from .race_common import build_planes_protos, soft_hash_probs


@dataclass
class GPTConfig:
    """The fields of chat/nanochat/gpt.py:36-52 that the attention layer reads."""
    sequence_len: int = 2048
    vocab_size: int = 32768
    n_layer: int = 12
    n_head: int = 6
    n_kv_head: int = 6
    n_embd: int = 768
    window_pattern: str = "SSSL"
    race_l: int = 3
    race_k: int = 3
    race_m: int = 1
    race_eps: float = 1e-6
    race_precision: str = "fp32"  # "fp32": gpt.py:132-140 exactly; "bf16": the fused kernels


def norm(x):
    """Parameter-free RMS norm over the last dim (gpt.py:55-56)."""
    return F.rms_norm(x, (x.size(-1),))


class Linear(nn.Linear):
    """Linear layer whose fp32 master weight is cast to the activation dtype (gpt.py:58-64)."""

    def forward(self, x):
        return F.linear(x, self.weight.to(dtype=x.dtype))


def apply_rotary_emb(x, cos, sin):
    """Rotate the two halves of the head dim by the position angle (gpt.py:71-77):
    x [B,T,H,D], cos/sin [1,T,1,D/2]."""
    half = x.shape[3] // 2
    a, b = x[..., :half], x[..., half:]
    return torch.cat([a * cos + b * sin, b * cos - a * sin], 3)


def rotary_tables(seq_len, head_dim, base=100000.0, device=None, dtype=torch.bfloat16):
    """cos, sin [1, seq_len, 1, head_dim/2] for apply_rotary_emb (gpt.py:273-286)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim))
    ang = torch.outer(torch.arange(seq_len, dtype=torch.float32, device=device), inv_freq)
    return ang.cos().to(dtype)[None, :, None, :], ang.sin().to(dtype)[None, :, None, :]


class RaceStateCache:
    """KV cache of a RACE model: one RaceDecodeState per layer plus the position.

    get_pos() and prev_embedding follow the cache interface GPT.forward uses
    (gpt.py:447, 463-465). The last attention layer of a forward advances the position.
    """

    def __init__(self, n_layer, batch, n_head, n_kv_head, head_dim, race_l, race_k, planes, eps=1e-6,
                 device="cuda"):
        self.n_layer = n_layer
        self.layers = [RaceDecodeState(batch, n_head, n_kv_head, head_dim, race_l, race_k, planes[i], eps=eps,
                                       device=device) for i in range(n_layer)]
        self.pos = 0
        self.prev_embedding = None

    def get_pos(self):
        return self.pos

    def advance(self, n):
        self.pos += n

    def reset(self):
        for st in self.layers:
            st.reset()
        self.pos = 0
        self.prev_embedding = None


def race_attend_fp32(q, k, v, planes_T, protos_T, L, Kbits, eps):
    """The reference seam's attention core (gpt.py:132-140) on [B,T,H,D] activations: fp32
    soft-hash (fp32 planes) and fp32 causal scan on the HIP kernels, k and v repeated over each
    query-head group; returns y [B,T,Hq,D] in q's dtype."""
    B, T, Hq, D = q.shape
    rep = Hq // k.shape[2]
    qf = q.transpose(1, 2).contiguous().float()
    kf = k.transpose(1, 2).contiguous().float()
    vf = v.transpose(1, 2).contiguous().float()
    if rep > 1:
        kf, vf = kf.repeat_interleave(rep, 1), vf.repeat_interleave(rep, 1)
    probsK, probsQ, V2, N = soft_hash_probs(qf, kf, vf, planes_T, protos_T, L, Kbits, 1, True)
    y = RaceCausalFn.apply(probsK, probsQ, V2, eps).view(B, Hq, T, D)
    return y.transpose(1, 2).to(q.dtype)


def race_attend(q, k, v, planes_T, L, Kbits, eps, state=None, precision="bf16", protos_T=None):
    """Causal RACE over [B,T,H,D] activations: q with Hq heads, k/v with Hkv heads.

    state None: the whole sequence, autograd-capable: precision "bf16" runs the fused kernels,
      "fp32" the reference's fp32 soft-hash + scan (race_attend_fp32; needs protos_T).
    state fresh and T > 1: prefill (fused); the state is left at the end of the sequence.
    otherwise: one decode step per token, updating the state in place.
    Returns y [B,T,Hq,D] in q's dtype.
    """
    if state is None and precision == "fp32":
        return race_attend_fp32(q, k, v, planes_T, protos_T, L, Kbits, eps)
    if precision not in ("fp32", "bf16"):
        raise ValueError(f"race precision must be 'fp32' or 'bf16', got {precision!r}")
    qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    if state is None:
        return race_causal_attention(qt, kt, vt, planes_T, L, Kbits, eps=eps, out_dtype=q.dtype).transpose(1, 2)
    if state.tokens == 0 and q.shape[1] > 1:
        return state.prefill(qt, kt, vt, out_dtype=q.dtype).transpose(1, 2)
    ys = [state.step(q[:, t].contiguous(), k[:, t].contiguous(), v[:, t].contiguous()) for t in range(q.shape[1])]
    return torch.stack(ys, 1)


def has_ve(layer_idx, n_layer):
    """Value embedding on alternating layers, the last one included (gpt.py:67-69)."""
    return layer_idx % 2 == (n_layer - 1) % 2


class CausalSelfAttention(nn.Module):
    """Drop-in for chat/nanochat/gpt.py:81-151 with grouped-query attention and a KV cache."""

    def __init__(self, config, layer_idx):
        super().__init__()
        self.layer_idx = layer_idx
        self.n_layer = config.n_layer
        self.n_head = config.n_head
        self.n_kv_head = config.n_kv_head
        self.n_embd = config.n_embd
        self.head_dim = self.n_embd // self.n_head
        if self.n_embd % self.n_head or self.n_head % self.n_kv_head or self.n_kv_head > self.n_head:
            raise ValueError("n_embd must split into n_head heads and n_head into n_kv_head groups")
        self.c_q = Linear(self.n_embd, self.n_head * self.head_dim, bias=False)
        self.c_k = Linear(self.n_embd, self.n_kv_head * self.head_dim, bias=False)
        self.c_v = Linear(self.n_embd, self.n_kv_head * self.head_dim, bias=False)
        self.c_proj = Linear(self.n_embd, self.n_embd, bias=False)
        self.ve_gate_channels = 12
        self.ve_gate = (Linear(self.ve_gate_channels, self.n_kv_head, bias=False)
                        if has_ve(layer_idx, config.n_layer) else None)
        self.race_L = config.race_l
        self.race_K = config.race_k
        self.race_M = config.race_m
        self.race_eps = config.race_eps
        self.race_precision = config.race_precision
        self.race_share_planes = True
        self.register_buffer("planes_T", torch.empty(self.head_dim, self.race_L * self.race_K))
        self.register_buffer("protos_T", torch.empty(self.race_K, 1 << self.race_K))

    @torch.no_grad()
    def init_race_buffers(self, seed=None):
        """planes/protos from build_planes_protos with seed = layer index (gpt.py:254-262)."""
        pl, pr = build_planes_protos(self.head_dim, self.race_K, self.race_L, self.race_M,
                                     device=self.planes_T.device, share_planes=True,
                                     seed=self.layer_idx if seed is None else seed)
        self.planes_T.copy_(pl)
        self.protos_T.copy_(pr)

    def forward(self, x, ve, cos_sin, window_size, kv_cache):
        B, T, _ = x.size()
        q = self.c_q(x).view(B, T, self.n_head, self.head_dim)
        k = self.c_k(x).view(B, T, self.n_kv_head, self.head_dim)
        v = self.c_v(x).view(B, T, self.n_kv_head, self.head_dim)
        if ve is not None:
            ve = ve.view(B, T, self.n_kv_head, self.head_dim)
            gate = 3 * torch.sigmoid(self.ve_gate(x[..., :self.ve_gate_channels]))
            v = v + gate.unsqueeze(-1) * ve
        cos, sin = cos_sin
        q, k = apply_rotary_emb(q, cos, sin), apply_rotary_emb(k, cos, sin)
        q, k = norm(q) * 1.2, norm(k) * 1.2
        # RACE has no sliding window: window_size is ignored, as in the reference (gpt.py:132)
        state = None if kv_cache is None else kv_cache.layers[self.layer_idx]
        y = race_attend(q, k, v, self.planes_T, self.race_L, self.race_K, self.race_eps, state,
                        precision=self.race_precision, protos_T=self.protos_T)
        if kv_cache is not None and self.layer_idx == self.n_layer - 1:
            kv_cache.advance(T)
        return self.c_proj(y.reshape(B, T, -1))


def make_cache(model_layers, batch, device="cuda"):
    """RaceStateCache for a list of CausalSelfAttention layers (one per block)."""
    a = model_layers[0]
    return RaceStateCache(len(model_layers), batch, a.n_head, a.n_kv_head, a.head_dim, a.race_L, a.race_K,
                          [m.planes_T for m in model_layers], eps=a.race_eps, device=device)
