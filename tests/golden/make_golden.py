"""Write golden vectors for soft_hash_probs from the reference itself.

Run in the build container only (the reference tree does not exist on the GPU
box): python tests/golden/make_golden.py

Why an import is needed: the fp32 soft-hash math is pinned by closed forms in
tests/test_oracle.py, but the reference's bf16 path rounds planes, the
projection, tanh and the logits to bf16 before its fp32 softmax
(scaling/race_common.py:54,65-72); nothing but the reference fixes those
roundings. This script imports scaling/race_common.py (torch only) and records
inputs and outputs of build_planes_protos + soft_hash_probs for a few small
cases, fp32 and bf16, into soft_hash_golden.npz (plain arrays, no pickle).
"""
import os
import sys

import numpy as np
import torch

REF = os.environ.get("RACE_REFERENCE_DIR", "/root/reference")
sys.path.insert(0, os.path.join(REF, "scaling"))
import race_common  # noqa: E402

CASES = [  # (B, H, T, D, L, Kbits, seed, dtype)
    (1, 2, 16, 16, 2, 2, 0, "float32"),
    (1, 2, 32, 64, 8, 4, 1, "float32"),
    (2, 1, 8, 64, 16, 4, 2, "float32"),
    (1, 2, 32, 64, 8, 4, 1, "bfloat16"),
    (2, 1, 8, 64, 16, 4, 2, "bfloat16"),
    (1, 1, 16, 128, 3, 3, 3, "bfloat16"),
]


def main():
    out = {}
    for i, (B, H, T, D, L, Kb, seed, dt) in enumerate(CASES):
        dtype = getattr(torch, dt)
        g = torch.Generator().manual_seed(100 + i)
        Q = torch.randn(B, H, T, D, generator=g).to(dtype)
        K = torch.randn(B, H, T, D, generator=g).to(dtype)
        V = torch.randn(B, H, T, D, generator=g).to(dtype)
        planes_T, protos_T = race_common.build_planes_protos(D, Kb, L, 1, device="cpu", seed=seed)
        pK, pQ, V2, N = race_common.soft_hash_probs(Q, K, V, planes_T, protos_T, L, Kb, 1, True)
        p = f"c{i}_"
        out[p + "meta"] = np.array([B, H, T, D, L, Kb, seed, int(dt == "bfloat16")], dtype=np.int64)
        out[p + "Q"] = Q.float().numpy()
        out[p + "K"] = K.float().numpy()
        out[p + "V"] = V.float().numpy()
        out[p + "planes_T"] = planes_T.numpy()
        out[p + "protos_T"] = protos_T.numpy()
        out[p + "probsK"] = pK.float().numpy()
        out[p + "probsQ"] = pQ.float().numpy()
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "soft_hash_golden.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
