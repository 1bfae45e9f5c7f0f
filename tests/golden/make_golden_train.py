"""Writes tests/golden/golden_train.npz: one training step of the reference SwiFFN_MoE.

    python tests/golden/make_golden_train.py

Run in the build container only (the reference is not present on the GPU box).
The reference layer (model.py:506-585) at d=128, h=320, E=4, top-2, tile 64,
in train mode with bf16 activations, through the reference CPU backend whose
fp8_forward and fp8_backward_input are the reference's own kernel/fp8_cpu.cpp
built under oracle/_ref (its JIT loader is never run).  One step: out =
moe(x), loss = sum(out.float() * c), loss.backward().

Stored (inputs and expected outputs only): x (bf16 as int16 bits), c, the
router weight, every expert's w8 / sc, the layer output, last_topi and the
token counts, x.grad (bf16 bits), gate.weight.grad (fp32), and every
executed expert's accumulated weight gradient _gw for gate / up / down (bf16
bits, kernel/fp8_tile.py:172-197; zeros and a flag 0 for an expert that did
not run).  A second step with the same x and c is taken, so _gw holds the sum
of two backward passes (the blockwise accumulation into bf16).
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

from make_golden import _backend, _np, ref_fp8, ref_model  # noqa: E402

D, E, K, TILE = 128, 4, 2, 64
B, T = 2, 40


def main():
    _backend()
    cfg = ref_model.LinearConfig(d_model=D, ffn_mult=2.5, tile=TILE, is_moe=True, num_experts=E,
                                 num_experts_per_tok=K, precision="fp8", architecture="plain")
    torch.manual_seed(0)
    moe = ref_model.SwiFFN_MoE(cfg).train()
    h = int(D * cfg.ffn_mult)
    g = torch.Generator().manual_seed(4711)
    out = {}
    with torch.no_grad():
        moe.gate.weight.copy_(torch.randn(E, D, generator=g) * 0.1)
        for e, ex in enumerate(moe.experts):
            for name, (o, i) in (("gate", (h, D)), ("up", (h, D)), ("down", (D, h))):
                lin = getattr(ex, name)
                w8, sc = ref_fp8.quantize_tiles(torch.randn(o, i, generator=g) * 0.05, TILE)
                lin.w8.copy_(w8)
                lin.sc.copy_(sc)
                out[f"e{e}_{name}_w8"] = _np(lin.w8).copy()
                out[f"e{e}_{name}_sc"] = _np(lin.sc).copy()
    x0 = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    c = torch.randn(B, T, D, generator=g)
    out["gate_w"] = _np(moe.gate.weight).copy()
    out["x"] = _np(x0).copy()
    out["c"] = _np(c).copy()
    for step in range(2):
        x = x0.clone().requires_grad_(True)
        y = moe(x)
        (y.float() * c).sum().backward()
        if step == 0:
            out["out"] = _np(y).copy()
            out["topi"] = _np(moe.last_topi).copy()
            out["counts"] = np.array(moe.expert_token_counts, dtype=np.int64)
            out["x_grad"] = _np(x.grad).copy()
            out["gate_grad"] = _np(moe.gate.weight.grad).copy()
    for e, ex in enumerate(moe.experts):
        for name in ("gate", "up", "down"):
            gw = getattr(ex, name)._gw
            out[f"e{e}_{name}_gw_ran"] = np.array(gw is not None)
            if gw is not None:
                assert gw.dtype == torch.bfloat16
                out[f"e{e}_{name}_gw"] = _np(gw).copy()
    path = os.path.join(HERE, "golden_train.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes; counts", out["counts"].tolist())


if __name__ == "__main__":
    main()
