"""Writes tests/golden/c5_skew.json: the router bias of config 5 (the large skewed layer).

    python tests/golden/make_c5_skew.py

Config 5: T=65536 tokens, d=2048, h=5120, E=16
experts, top-2, x ~ N(0,1) cast to bf16 once, router weight N(0,0.02).  The
router bias is zero except b[0] = +beta_hi and b[13..15] = -beta_lo.  Both
betas are found by bisection on the first 4096 tokens so that expert 0 holds
39-41 % of the T*k assignments and experts 13-15 each hold under 1 %.

The routing is model.py:558-570 (fp32 logits, softmax, top-k, renorm), taken
from the CPU oracle; the bisection itself is plain arithmetic on its counts.
Inputs are drawn on the CPU from one torch.Generator seeded 1234 + 4 in the
order x, router W, router b (drawn, then replaced by the skew bias), so the
GPU tests regenerate the same x and W from the seed alone.
"""
import json
import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

import oracle  # noqa: E402

SEED = 1234 + 4
T, D, H, E, K = 65536, 2048, 5120, 16, 2
LOW = (13, 14, 15)
N_FIT = 4096


def draw_router_inputs(n_tokens=T):
    """x [n_tokens, D] (bf16) and router W [E, D] fp32 from the config-5 seed."""
    gen = torch.Generator().manual_seed(SEED)
    x = torch.randn(T, D, generator=gen)[:n_tokens]
    w = torch.randn(E, D, generator=gen) * 0.02
    torch.randn(E, generator=gen)  # the drawn bias, replaced by skew_bias()
    return x.to(torch.bfloat16), w


def skew_bias(beta_hi, beta_lo):
    b = torch.zeros(E)
    b[0] = beta_hi
    for e in LOW:
        b[e] = -beta_lo
    return b


def shares(x, w, beta_hi, beta_lo):
    _, topi, topw = oracle.route(x, w, skew_bias(beta_hi, beta_lo), K)
    counts = [int(((topi == e) & (topw > 0)).any(-1).sum()) for e in range(E)]
    tot = x.shape[0] * K
    return [c / tot for c in counts], counts


def bisect(f, lo, hi, want, iters=40):
    """Root of the increasing function f(beta) - want on [lo, hi]."""
    for _ in range(iters):
        mid = 0.5 * (lo + hi)
        if f(mid) < want:
            lo = mid
        else:
            hi = mid
    return 0.5 * (lo + hi)


def main():
    x, w = draw_router_inputs(N_FIT)
    beta_lo = 0.0
    beta_hi = 0.0
    for _ in range(3):  # the two biases interact weakly: alternate until both hold
        beta_lo = bisect(lambda b: -max(shares(x, w, beta_hi, b)[0][e] for e in LOW), 0.0, 16.0, -0.005)
        beta_hi = bisect(lambda b: shares(x, w, b, beta_lo)[0][0], 0.0, 16.0, 0.40)
    fr, counts = shares(x, w, beta_hi, beta_lo)
    assert 0.39 <= fr[0] <= 0.41, fr
    assert all(fr[e] < 0.01 for e in LOW), fr
    out = {
        "config": "C5: T=65536 d=2048 h=5120 E=16 top-2 tile 64",
        "seed": SEED,
        "draw_order": "x [65536,2048] N(0,1), router W [16,2048] N(0,0.02), router b [16] (replaced)",
        "beta_hi": beta_hi,
        "beta_lo": beta_lo,
        "bias_rule": "b = 0; b[0] = +beta_hi; b[13], b[14], b[15] = -beta_lo",
        "fit_tokens": N_FIT,
        "fit_counts": counts,
        "fit_share_e0": fr[0],
        "fit_share_low": [fr[e] for e in LOW],
    }
    path = os.path.join(HERE, "c5_skew.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(json.dumps(out, indent=1))


if __name__ == "__main__":
    main()
