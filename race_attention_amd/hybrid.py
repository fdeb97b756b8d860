"""Llama-3.2-1B-shaped language model with RACE attention in every layer (random init).

A workload model for the hybrid integration, not a reference component: 16 layers,
hidden 2048, 32 query / 8 kv heads of dim 64, rotary embeddings, SwiGLU MLP 8192, RMS
norms, untied embedding and head, RACE (L=8, K=4) attention through the fused bf16
kernels. Prefill runs the fused forward (and backward when training); generation carries
one RACE bucket state per layer (RaceStateCache) and decodes each token with one
race_decode_step kernel per layer, where the reference re-runs the whole forward per
token (chat/nanochat/gpt.py:514-544).
"""
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from .nanochat import Linear, RaceStateCache, apply_rotary_emb, race_attend, rotary_tables
from .race_common import build_planes_protos


@dataclass
class HybridConfig:
    vocab_size: int = 128256
    n_layer: int = 16
    n_embd: int = 2048
    n_head: int = 32
    n_kv_head: int = 8
    mlp_hidden: int = 8192
    max_seq_len: int = 8192 + 512
    rope_base: float = 500000.0
    norm_eps: float = 1e-5
    race_l: int = 8
    race_k: int = 4
    race_eps: float = 1e-6
    # logits from an fp32 product of the final hidden state and the head weights (else the head
    # runs in the weights' dtype and its bf16-rounded logits tie often in a small random model)
    fp32_logits: bool = False


class RMSNorm(nn.Module):
    def __init__(self, dim, eps):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        return F.rms_norm(x, (x.size(-1),), self.weight.to(x.dtype), self.eps)


class RaceSelfAttention(nn.Module):
    def __init__(self, cfg, layer_idx):
        super().__init__()
        self.layer_idx, self.n_layer = layer_idx, cfg.n_layer
        self.n_head, self.n_kv_head = cfg.n_head, cfg.n_kv_head
        self.head_dim = cfg.n_embd // cfg.n_head
        self.L, self.K, self.eps = cfg.race_l, cfg.race_k, cfg.race_eps
        self.q_proj = Linear(cfg.n_embd, cfg.n_head * self.head_dim, bias=False)
        self.k_proj = Linear(cfg.n_embd, cfg.n_kv_head * self.head_dim, bias=False)
        self.v_proj = Linear(cfg.n_embd, cfg.n_kv_head * self.head_dim, bias=False)
        self.o_proj = Linear(cfg.n_head * self.head_dim, cfg.n_embd, bias=False)
        self.register_buffer("planes_T", torch.empty(self.head_dim, self.L * self.K))

    def forward(self, x, cos_sin, cache=None):
        B, T, _ = x.shape
        q = self.q_proj(x).view(B, T, self.n_head, self.head_dim)
        k = self.k_proj(x).view(B, T, self.n_kv_head, self.head_dim)
        v = self.v_proj(x).view(B, T, self.n_kv_head, self.head_dim)
        cos, sin = cos_sin
        q, k = apply_rotary_emb(q, cos, sin), apply_rotary_emb(k, cos, sin)
        state = None if cache is None else cache.layers[self.layer_idx]
        y = race_attend(q, k, v, self.planes_T, self.L, self.K, self.eps, state)
        if cache is not None and self.layer_idx == self.n_layer - 1:
            cache.advance(T)
        return self.o_proj(y.reshape(B, T, -1))


class SwiGLU(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.gate = Linear(cfg.n_embd, cfg.mlp_hidden, bias=False)
        self.up = Linear(cfg.n_embd, cfg.mlp_hidden, bias=False)
        self.down = Linear(cfg.mlp_hidden, cfg.n_embd, bias=False)

    def forward(self, x):
        return self.down(F.silu(self.gate(x)) * self.up(x))


class Block(nn.Module):
    def __init__(self, cfg, layer_idx):
        super().__init__()
        self.norm1 = RMSNorm(cfg.n_embd, cfg.norm_eps)
        self.attn = RaceSelfAttention(cfg, layer_idx)
        self.norm2 = RMSNorm(cfg.n_embd, cfg.norm_eps)
        self.mlp = SwiGLU(cfg)

    def forward(self, x, cos_sin, cache=None):
        x = x + self.attn(self.norm1(x), cos_sin, cache)
        return x + self.mlp(self.norm2(x))


class HybridLM(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab_size, cfg.n_embd)
        self.blocks = nn.ModuleList([Block(cfg, i) for i in range(cfg.n_layer)])
        self.norm = RMSNorm(cfg.n_embd, cfg.norm_eps)
        self.lm_head = Linear(cfg.n_embd, cfg.vocab_size, bias=False)
        cos, sin = rotary_tables(cfg.max_seq_len, cfg.n_embd // cfg.n_head, cfg.rope_base)
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)

    @torch.no_grad()
    def init_weights(self, seed=0, dtype=torch.bfloat16):
        """Random init (normal, std 0.02; output projections scaled by 1/sqrt(2*n_layer)),
        RACE planes seeded by layer index, weights cast to `dtype`."""
        dev = self.embed.weight.device
        g = torch.Generator(device=dev).manual_seed(seed)
        for name, p in self.named_parameters():
            if name.endswith("norm1.weight") or name.endswith("norm2.weight") or name == "norm.weight":
                p.fill_(1.0)
                continue
            std = 0.02 / (2 * self.cfg.n_layer) ** 0.5 if name.endswith(("o_proj.weight", "down.weight")) else 0.02
            p.copy_(torch.randn(p.shape, generator=g, device=dev) * std)
        for i, blk in enumerate(self.blocks):
            pl, _ = build_planes_protos(blk.attn.head_dim, self.cfg.race_k, self.cfg.race_l, 1,
                                        device=blk.attn.planes_T.device, seed=i)
            blk.attn.planes_T.copy_(pl)
        self.to(dtype)
        for blk in self.blocks:
            blk.attn.planes_T.data = blk.attn.planes_T.float()
        cos, sin = rotary_tables(self.cfg.max_seq_len, self.cfg.n_embd // self.cfg.n_head, self.cfg.rope_base,
                                 device=self.cos.device, dtype=dtype)
        self.cos, self.sin = cos, sin
        return self

    def make_cache(self, batch):
        a = self.blocks[0].attn
        return RaceStateCache(self.cfg.n_layer, batch, a.n_head, a.n_kv_head, a.head_dim, a.L, a.K,
                              [b.attn.planes_T for b in self.blocks], eps=a.eps, device=self.embed.weight.device)

    def forward(self, idx, cache=None, targets=None, pos=None):
        """idx [B, T] token ids. With a cache the sequence continues at cache.get_pos(), or at the
        device tensor `pos` ([1], int64) when given: a captured decode step reads its rotary
        rows through it, so one HIP graph serves every position."""
        B, T = idx.shape
        if pos is None:
            t0 = 0 if cache is None else cache.get_pos()
            self.check_length(t0 + T)
            cos_sin = self.cos[:, t0:t0 + T], self.sin[:, t0:t0 + T]
        else:
            rows = pos + torch.arange(T, device=pos.device)
            cos_sin = self.cos.index_select(1, rows), self.sin.index_select(1, rows)
        x = self.embed(idx)
        for blk in self.blocks:
            x = blk(x, cos_sin, cache)
        if self.cfg.fp32_logits:
            logits = F.linear(self.norm(x).float(), self.lm_head.weight.float())
        else:
            logits = self.lm_head(self.norm(x)).float()
        if targets is None:
            return logits
        return F.cross_entropy(logits.reshape(-1, logits.size(-1)), targets.reshape(-1))

    def check_length(self, total):
        """Rotary tables cover cfg.max_seq_len positions: longer sequences are refused on the
        host (a captured decode step reads its rows through a device-side position)."""
        if total > self.cfg.max_seq_len:
            raise ValueError(f"sequence of {total} tokens exceeds max_seq_len = {self.cfg.max_seq_len}")

    @torch.no_grad()
    def generate_graphed(self, idx, n_new):
        """Greedy decode as generate(idx, n_new), each token step one replay of a captured HIP
        graph (GraphedDecoder). Returns the same (tokens, logits) pair."""
        self.check_length(idx.shape[1] + n_new - 1)  # the last token is not fed back
        dec = GraphedDecoder(self, idx)
        for _ in range(n_new - 1):
            dec.step()
        return dec.finish()

    @torch.no_grad()
    def generate(self, idx, n_new, use_cache=True):
        """Greedy decode: returns (tokens [B, n_new], per-step last-position logits [n_new, B, V]).
        use_cache=False re-runs the full forward per token (the reference's GPT.generate)."""
        self.check_length(idx.shape[1] + n_new - 1)  # the last token is not fed back
        toks, steps = [], []
        if use_cache:
            cache = self.make_cache(idx.shape[0])
            logits = self.forward(idx, cache)[:, -1]
            for i in range(n_new):
                nxt = logits.argmax(-1, keepdim=True)
                toks.append(nxt)
                steps.append(logits)
                if i + 1 < n_new:
                    logits = self.forward(nxt, cache)[:, -1]
        else:
            seq = idx
            for _ in range(n_new):
                logits = self.forward(seq)[:, -1]
                nxt = logits.argmax(-1, keepdim=True)
                toks.append(nxt)
                steps.append(logits)
                seq = torch.cat([seq, nxt], 1)
        return torch.cat(toks, 1), torch.stack(steps)


class GraphedDecoder:
    """Greedy decoding of a HybridLM with one captured HIP graph per token step.

    The constructor prefills a RaceStateCache eagerly from idx [B, T0] and picks the first token;
    it then captures one step — embedding, the blocks (one fused RACE decode kernel each), the
    head, the argmax that feeds the next step's token and the position increment, the position
    living in a device tensor so one graph serves every step. step() replays it: no host work
    per token beyond the replay. finish() returns (tokens [B, n], logits [n, B, V]) as
    HybridLM.generate does, and leaves the cache's counters at the decoded length.
    """

    @torch.no_grad()
    def __init__(self, model, idx):
        self.model = model
        B = idx.shape[0]
        # the capture itself runs one step past the prompt (on a throwaway cache)
        model.check_length(idx.shape[1] + 1)
        self.cache = model.make_cache(B)
        logits = model(idx, self.cache)[:, -1]
        self.tok = logits.argmax(-1, keepdim=True)
        self.toks, self.steps = [self.tok.clone()], [logits.clone()]
        self.pos = torch.tensor([self.cache.get_pos()], dtype=torch.long, device=idx.device)
        # lazy library state (BLAS handles and workspaces, code objects) is set up by one run on
        # a throwaway cache, on a side stream, before the capture; the real cache is not touched
        scratch = model.make_cache(B)
        tok0, pos0 = self.tok.clone(), self.pos.clone()
        side = torch.cuda.Stream(device=idx.device)
        side.wait_stream(torch.cuda.current_stream(idx.device))
        with torch.cuda.stream(side):
            self._step(scratch)
        torch.cuda.current_stream(idx.device).wait_stream(side)
        self.tok.copy_(tok0)
        self.pos.copy_(pos0)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = self._step(self.cache)
        # the capture ran the step's host side once without its kernels: undo its counters
        self.cache.pos -= 1
        for st in self.cache.layers:
            st.tokens -= 1
        self.n = 0

    def _step(self, cache):
        out = self.model(self.tok, cache, pos=self.pos)[:, -1]
        self.tok.copy_(out.argmax(-1, keepdim=True))
        self.pos.add_(1)
        return out

    def step(self, keep=True):
        """One token for every sequence (kept for finish() unless keep=False). Refused on the
        host once the position would pass the rotary tables (cfg.max_seq_len)."""
        self.model.check_length(self.cache.pos + self.n + 1)
        self.graph.replay()
        self.n += 1
        if keep:
            self.toks.append(self.tok.clone())
            self.steps.append(self.out.clone())

    def finish(self):
        self.cache.pos += self.n
        for st in self.cache.layers:
            st.tokens += self.n
        self.n = 0
        return torch.cat(self.toks, 1), torch.stack(self.steps)
