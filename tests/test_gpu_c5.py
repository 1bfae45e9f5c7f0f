"""Config 5 at full size: the large skewed MoE layer.

T=65536 tokens, d=2048, h=5120, E=16 experts, top-2, tile 64, bf16
activations.  The router bias puts ~40 % of the assignments on expert 0 and
under 1 % on each of experts 13-15; its two values were found by bisection on
the first 4096 tokens (tests/golden/make_c5_skew.py -> c5_skew.json).

Bars: top-k indices and per-expert counts of all
65536 tokens bit-exact against the oracle router (model.py:558-570 on the
CPU), and rel-L2 <= 2e-3 of the layer output against the oracle's
model.py:557-585 loop on a token sample (tokens are independent).
"""
import json
import os

import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
DEV = "cuda"
T, D, H, E, K = 65536, 2048, 5120, 16, 2


def c5_inputs():
    """x (bf16, CPU), router W and the skew bias, regenerated from the committed seed."""
    cfg = json.load(open(os.path.join(HERE, "golden", "c5_skew.json")))
    gen = torch.Generator().manual_seed(cfg["seed"])
    x = torch.randn(T, D, generator=gen).to(torch.bfloat16)
    w = torch.randn(E, D, generator=gen) * 0.02
    b = torch.zeros(E)
    b[0] = cfg["beta_hi"]
    for e in (13, 14, 15):
        b[e] = -cfg["beta_lo"]
    return x, w, b


def device_experts(seed, tile=64):
    """E experts drawn N(0, 0.02) on the device and quantized to tiled E4M3 there
    (the same quantizer as on the host; only the draw differs)."""
    from smaulnative_amd.fp8_tile import quantize_tiles
    gen = torch.Generator(device=DEV).manual_seed(seed)
    out = []
    for _ in range(E):
        parts = []
        for (o, i) in ((H, D), (H, D), (D, H)):
            w8, sc = quantize_tiles(torch.randn(o, i, generator=gen, device=DEV) * 0.02, tile)
            parts += [w8, sc]
        out.append(tuple(parts))
    return out


def test_c5_full_size_routing_and_output():
    from smaulnative_amd.compute import get_backend
    print("case C5 T=65536 d=2048 h=5120 E=16 k=2", flush=True)
    x, w, b = c5_inputs()
    prob_r, topi_r, topw_r = oracle.route(x, w, b, K)
    counts_r = [int(((topi_r == e) & (topw_r > 0)).any(-1).sum()) for e in range(E)]
    exd = device_experts(1238)
    be = get_backend("rocm")
    out, prob, topi, counts = be.moe_forward(x.to(DEV), w.to(DEV), b.to(DEV), exd, K, 64)
    torch.cuda.synchronize()
    topi, counts, prob = topi.cpu(), counts.cpu().tolist(), prob.cpu()
    flips = int((topi != topi_r).any(-1).sum())
    print(f"counts {counts} flips {flips}", flush=True)
    # every token's routing, bit for bit
    assert torch.equal(topi, topi_r)
    assert counts == counts_r
    assert float(((prob - prob_r).abs() / prob_r.abs().clamp_min(1e-30)).max()) < 1e-5
    # the skew the config asks for, over the whole layer
    assert 0.38 <= counts[0] / (T * K) <= 0.42
    assert all(counts[e] / (T * K) < 0.01 for e in (13, 14, 15))
    # the output of a token sample against the oracle's expert loop
    idx = torch.arange(0, T, 257)
    experts = [oracle.ExpertWeights(*[t.cpu() for t in ex]) for ex in exd]
    ref = oracle.moe_forward(x[idx], w, b, experts, K, 64)
    assert torch.equal(ref.topi, topi_r[idx])
    o = out[idx.to(DEV)].cpu().double()
    r = ref.out.double()
    err = float((o - r).norm() / r.norm())
    print(f"rel_l2 {err:.3e} on {idx.numel()} tokens", flush=True)
    assert err < 2e-3
