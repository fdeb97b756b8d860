"""Fused single-token decode with carried RACE state.

The reference has no decode path (chat/nanochat/gpt.py:143-146 raises and
GPT.generate re-runs the full forward per token, gpt.py:533-534). The state of a
causal RACE layer after t tokens is exactly race_prefix_ref's (A_final, B_final)
(scaling/race_common.py:88-90): A [S] = sum pK, B [S,D] = sum pK v. Decoding a
token updates it in place (A += pK, B += pK v^T) and reads out
out = sum_s pQ[s] B[s,:] / (A[s] + eps) for every query head of the group, in one
HIP kernel per step (race_decode_step).
"""
import math

import torch

from . import _lib
from .attention import race_causal_attention_with_state


class RaceDecodeState:
    """Per-layer decode state for B sequences and Hkv kv heads (fp32, HBM-resident).

    A  [B*Hkv, S]     running sum of key bucket probabilities
    Bs [B*Hkv, S, D]  running sum of pK (x) v
    """

    def __init__(self, B, Hq, Hkv, D, L, Kbits, planes_T, scale=None, eps=1e-6, device="cuda"):
        if Hq % Hkv:
            raise ValueError("Hq must be a multiple of Hkv")
        self.B, self.Hq, self.Hkv, self.D, self.L, self.K = B, Hq, Hkv, D, L, Kbits
        self.S = L << Kbits
        self.scale = math.sqrt(D) if scale is None else float(scale)
        self.eps = float(eps)
        self.planes = planes_T.detach().float().contiguous().to(device)
        self.A = torch.zeros(B * Hkv, self.S, dtype=torch.float32, device=device)
        self.Bs = torch.zeros(B * Hkv, self.S, D, dtype=torch.float32, device=device)
        self.tokens = 0

    def reset(self):
        self.A.zero_()
        self.Bs.zero_()
        self.tokens = 0

    def prefill(self, q, k, v, out_dtype=None):
        """Causal RACE over a prompt (q [B,Hq,T,D], k/v [B,Hkv,T,D] bf16) that also
        leaves this state at the end of the prompt. Returns the prompt's output.
        The state must be fresh (prefill starts from zero)."""
        if self.tokens:
            raise RuntimeError("prefill on a non-empty state; call reset() first")
        out, A, Bs = race_causal_attention_with_state(q, k, v, self.planes, self.L, self.K, self.scale,
                                                      self.eps, out_dtype)
        self.A.copy_(A)
        self.Bs.copy_(Bs)
        self.tokens = q.shape[2]
        return out

    def step(self, q, k, v, out=None):
        """One token per sequence: q [B,Hq,D], k/v [B,Hkv,D] (bf16 or fp32) -> out [B,Hq,D]."""
        _lib.require_device(q, k, v)
        if q.shape != (self.B, self.Hq, self.D) or k.shape != (self.B, self.Hkv, self.D) or v.shape != k.shape:
            raise ValueError(f"step expects q [{self.B},{self.Hq},{self.D}] and k/v [{self.B},{self.Hkv},{self.D}]")
        if not (q.dtype == k.dtype == v.dtype):
            raise ValueError("q, k, v must share a dtype")
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        if out is None:
            out = torch.empty_like(q)
        sh = _lib.DecodeShape(self.B, self.Hq, self.Hkv, self.D, self.L, self.K, self.scale, self.eps)
        _lib.check(_lib.lib().race_decode_step(sh, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.dtype_code(q.dtype),
                                               _lib.ptr(self.planes), _lib.ptr(self.A), _lib.ptr(self.Bs),
                                               _lib.ptr(out), _lib.stream_of(q)), "race_decode_step")
        self.tokens += 1
        return out
