"""Shared loaders for the golden fixtures (tests/golden/golden_fp8_moe.npz)."""
import numpy as np
import torch

import oracle


def _t(a):
    return torch.from_numpy(np.array(a))


def _bf(a):
    return torch.from_numpy(np.array(a)).view(torch.bfloat16)


def load_moe_case(g, tag):
    d, E, k, tile, h = g[f"{tag}_meta"].tolist()
    is_bf16 = int(g[f"{tag}_dtype"][0]) == 1
    x = _bf(g[f"{tag}_x"]) if is_bf16 else _t(g[f"{tag}_x"])
    experts = []
    for e in range(E):
        parts = []
        for nm in ("gate", "up", "down"):
            parts += [_t(g[f"{tag}_e{e}_{nm}_w"]), _t(g[f"{tag}_e{e}_{nm}_s"])]
        experts.append(oracle.ExpertWeights(*parts))
    out = _bf(g[f"{tag}_out"]) if is_bf16 else _t(g[f"{tag}_out"])
    return dict(d=d, E=E, k=k, tile=tile, h=h, x=x, gate_w=_t(g[f"{tag}_gate_w"]), experts=experts,
                out=out, prob=_t(g[f"{tag}_prob"]), topi=_t(g[f"{tag}_topi"]),
                counts=g[f"{tag}_counts"].tolist(), executed=[bool(v) for v in g[f"{tag}_executed"]])


