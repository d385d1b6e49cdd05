"""Writes config1_reduced.npz: the acceptance inputs of BASELINE config 1
at a reduced vocabulary (8 sequences, k = 4, V = 2048, seed 0), drafts
planted as their row's maximum with probability 0.7 per position, and the
expected results computed here without the oracle: numpy's first-index
argmax over the bf16 values, and the first-mismatch scan of
nanovllm/engine/speculative.py:11-30 (accept length = drafts matched before
the first mismatch, bonus = the argmax of the row after them).

Run from the repository root: python tests/golden/gen_config1_fixture.py"""
import os

import numpy as np
import torch

B, K, V = 8, 4, 2048


def main() -> None:
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(B, K + 1, V, generator=g)
    prop = torch.randint(0, V, (B, K), generator=g)
    hit = torch.rand(B, K, generator=g) < 0.7
    for s in range(B):
        for j in range(K):
            if hit[s, j]:
                logits[s, j, prop[s, j]] = logits[s, j].max() + 1.0
    prev = torch.randint(0, V, (B, 1), generator=g)
    bf = logits.view(B * (K + 1), V).to(torch.bfloat16)
    bits = bf.view(torch.int16).numpy().view(np.uint16)
    values = bf.float().numpy()
    argmax = values.argmax(axis=1).astype(np.int32)          # first maximal index
    ids = torch.cat([prev, prop], 1).reshape(-1).numpy().astype(np.int64)
    accept = np.zeros(B, np.int32)
    bonus = np.zeros(B, np.int32)
    for s in range(B):
        rows = argmax[s * (K + 1):(s + 1) * (K + 1)]
        drafts = ids[s * (K + 1) + 1:(s + 1) * (K + 1)]
        a = 0
        while a < K and drafts[a] == rows[a]:
            a += 1
        accept[s], bonus[s] = a, rows[a]
    cu_q = np.arange(0, B * (K + 1) + 1, K + 1, dtype=np.int32)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "config1_reduced.npz")
    np.savez_compressed(out, logits_bits=bits, cu_q=cu_q, input_ids=ids, argmax=argmax,
                        accept_len=accept, bonus=bonus)
    print(out, "accept", accept.tolist(), "bonus", bonus.tolist())


if __name__ == "__main__":
    main()
