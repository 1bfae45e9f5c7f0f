"""Writes tests/golden/golden_attn.npz from the reference's own linear-attention kernel.

    python tests/golden/make_golden_attn.py

The kernel is kernel/attn_cpu.cpp compiled from source by oracle/Makefile into
oracle/_ref (its JIT loader is never run).  Cases: attn_forward with DEN and
the final state on ragged shapes (D = 13, 64, 130; T = 1, 5, 37), then one
attn_step from that state.  Inputs follow model.py's feature map: q and k are
elu(N(0,1)) + 1, v is N(0,1); one case has an all-zero key row (the 1e-6
clamp of attn_cpu.cpp:44-46) and one a large eps (the den clamp).  The states S are stored for the small
cases only; the step of the others starts from the state the forward returns.
"""
import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

import oracle  # noqa: E402  (only for oracle/_ref, the reference kernel build)

CASES = [  # (B, T, H, D, eps, zero_key)
    (1, 37, 2, 64, 1e-6, False),
    (1, 5, 2, 13, 1e-6, True),
    (1, 4, 1, 130, 1e-6, False),
    (2, 1, 2, 64, 1e-6, False),
    (1, 9, 2, 32, 5.0, False),
]
S_MAX = 8192  # the states are stored only for cases with B*H*D*D <= S_MAX (fixture size)


def main():
    mod = oracle.ref_attn_module()
    if mod is None:
        raise SystemExit("build oracle/_ref first: make -C oracle")
    g = torch.Generator().manual_seed(31)
    out = {"cases": np.array([c[:4] for c in CASES], dtype=np.int64),
           "eps": np.array([c[4] for c in CASES], dtype=np.float32)}
    for i, (B, T, H, D, eps, zk) in enumerate(CASES):
        Q = F.elu(torch.randn(B, T, H, D, generator=g)) + 1
        K = F.elu(torch.randn(B, T, H, D, generator=g)) + 1
        V = torch.randn(B, T, H, D, generator=g)
        if zk:
            K[0, 2, 1] = 0.0
        Y, DEN, S, z = mod.attn_forward(Q, K, V, eps, True, True)
        q = F.elu(torch.randn(B, H, D, generator=g)) + 1
        k = F.elu(torch.randn(B, H, D, generator=g)) + 1
        v = torch.randn(B, H, D, generator=g)
        S1, z1 = S.clone(), z.clone()
        y1, S1, z1 = mod.attn_step(S1, z1, q, k, v, eps)
        keep = [("Q", Q), ("K", K), ("V", V), ("Y", Y), ("DEN", DEN), ("z", z), ("q", q), ("k", k), ("v", v),
                ("y1", y1), ("z1", z1)]
        if B * H * D * D <= S_MAX:
            keep += [("S", S), ("S1", S1)]
        for name, t in keep:
            out[f"a{i}_{name}"] = t.numpy()
    path = os.path.join(HERE, "golden_attn.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
