"""Loading the MoE layers of a SmaulLinear checkpoint onto the device.

A checkpoint is a directory with ``config.json`` and ``model.safetensors``
(model.py:904-944, ``save_pretrained``).  Its MoE tensors follow the expert
layout ``merge_moe.py`` writes (merge_moe.py:110-119): a dense FFN tensor
``blocks.N.ffn.<proj>.<buf>`` becomes ``blocks.N.ffn.experts.E.<proj>.<buf>``,
beside the router ``blocks.N.ffn.gate.weight``:

    blocks.N.ffn.gate.weight                fp32 [E, d]
    blocks.N.ffn.experts.E.gate.w8 / .sc    uint8 [h, d] / fp32 [h, ceil(d/tile)]
    blocks.N.ffn.experts.E.up.w8 / .sc      uint8 [h, d] / fp32 [h, ceil(d/tile)]
    blocks.N.ffn.experts.E.down.w8 / .sc    uint8 [d, h] / fp32 [d, ceil(h/tile)]

``load_moe_layers`` reads only those tensors, one at a time and straight to
the device (safetensors' lazy reader), checks every key, shape and dtype the
config implies (the strict load of model.py:1004: a missing or unexpected
MoE tensor raises), restores scales stored in a narrower float dtype to fp32
as LinearInference does after a bf16 cast (inference.py:86-97), and builds
the rocm backend's repack cache for each layer (the canonical code copies,
0x7F/0xFF -> 0x7E/0xFE), so the first forward pays nothing.  The stored
``w8`` / ``sc`` are kept unchanged: the cache is refreshed whenever a buffer
is rewritten in place (requant, kernel/fp8_tile.py:252-253).
"""
from __future__ import annotations

import json
import os
import re
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch

PROJ = ("gate", "up", "down")
_EXPERT_KEY = re.compile(r"^blocks\.(\d+)\.ffn\.experts\.(\d+)\.(gate|up|down)\.(w8|sc)$")
_ROUTER_KEY = re.compile(r"^blocks\.(\d+)\.ffn\.gate\.(weight|bias)$")


@dataclass
class MoELayer:
    """One SwiFFN_MoE's weights on the device, in the reference's storage format."""
    index: int
    gate_weight: torch.Tensor                    # fp32 [E, d]
    gate_bias: Optional[torch.Tensor]            # fp32 [E] or None
    experts: List[Tuple[torch.Tensor, ...]] = field(default_factory=list)  # (gw8, gsc, uw8, usc, dw8, dsc)
    top_k: int = 1
    tile: int = 64

    def forward(self, x):
        """SwiFFN_MoE.forward of this layer on the rocm backend (see RocmBackend.moe_forward)."""
        from smaulnative_amd.compute import get_backend
        return get_backend("rocm").moe_forward(x, self.gate_weight, self.gate_bias, self.experts, self.top_k,
                                               self.tile)


def read_config(ckpt_dir) -> dict:
    with open(os.path.join(ckpt_dir, "config.json")) as f:
        cfg = json.load(f)
    for key in ("d_model", "ffn_mult", "tile", "num_experts", "num_experts_per_tok", "n_layer"):
        if key not in cfg:
            raise ValueError(f"{ckpt_dir}/config.json has no {key!r}")
    if not cfg.get("is_moe", False):
        raise ValueError(f"{ckpt_dir} is not a MoE checkpoint (is_moe is false)")
    if cfg.get("precision", "fp8") != "fp8":
        raise ValueError(f"{ckpt_dir}: the rocm MoE path loads precision='fp8' checkpoints only")
    if cfg.get("architecture", "plain") != "plain":
        raise ValueError(f"{ckpt_dir}: the rocm MoE path loads architecture='plain' checkpoints only")
    return cfg


def _expected(cfg) -> Dict[str, Tuple[Tuple[int, ...], torch.dtype]]:
    d, tile, E = int(cfg["d_model"]), int(cfg["tile"]), int(cfg["num_experts"])
    h = int(d * float(cfg["ffn_mult"]))
    nt_d, nt_h = -(-d // tile), -(-h // tile)
    shapes = {"gate": ((h, d), (h, nt_d)), "up": ((h, d), (h, nt_d)), "down": ((d, h), (d, nt_h))}
    want = {}
    for l in range(int(cfg["n_layer"])):
        want[f"blocks.{l}.ffn.gate.weight"] = ((E, d), torch.float32)
        for e in range(E):
            for p in PROJ:
                want[f"blocks.{l}.ffn.experts.{e}.{p}.w8"] = (shapes[p][0], torch.uint8)
                want[f"blocks.{l}.ffn.experts.{e}.{p}.sc"] = (shapes[p][1], torch.float32)
    return want


def load_moe_layers(ckpt_dir, device="cuda", layers=None, prepare=True) -> List[MoELayer]:
    """The MoE layers of the checkpoint in ``ckpt_dir`` on ``device`` (all, or those in ``layers``)."""
    from safetensors import safe_open
    cfg = read_config(ckpt_dir)
    want = _expected(cfg)
    path = os.path.join(ckpt_dir, "model.safetensors")
    dev = torch.device(device)
    tensors: Dict[str, torch.Tensor] = {}
    with safe_open(path, framework="pt", device=str(dev)) as f:
        keys = set(f.keys())
        moe_keys = {k for k in keys if _EXPERT_KEY.match(k) or _ROUTER_KEY.match(k)}
        stray = sorted(k for k in keys - moe_keys if ".ffn.experts." in k)
        missing = sorted(set(want) - keys)
        unexpected = sorted(k for k in moe_keys if k not in want and not k.endswith(".ffn.gate.bias"))
        if missing or unexpected or stray:
            raise RuntimeError(f"{path}: MoE tensors do not match config.json: missing {missing[:8]}, "
                               f"unexpected {(unexpected + stray)[:8]}")
        sel = None if layers is None else {int(l) for l in layers}
        for k in sorted(moe_keys):
            m = _EXPERT_KEY.match(k) or _ROUTER_KEY.match(k)
            if sel is not None and int(m.group(1)) not in sel:
                continue
            t = f.get_tensor(k)
            if k in want:
                shape, dtype = want[k]
                if tuple(t.shape) != shape:
                    raise RuntimeError(f"{path}: {k} has shape {tuple(t.shape)}, config implies {shape}")
                if dtype == torch.uint8 and t.dtype != torch.uint8:
                    raise RuntimeError(f"{path}: {k} must be uint8 codes, got {t.dtype}")
                if dtype == torch.float32 and not t.is_floating_point():
                    raise RuntimeError(f"{path}: {k} must be floating point, got {t.dtype}")
            if t.is_floating_point() and t.dtype != torch.float32:
                t = t.float()   # a bf16-cast checkpoint: scales and router back to fp32 (inference.py:86-97)
            tensors[k] = t.contiguous()
    E, k_top, tile = int(cfg["num_experts"]), int(cfg["num_experts_per_tok"]), int(cfg["tile"])
    d = int(cfg["d_model"])
    h = int(d * float(cfg["ffn_mult"]))
    out = []
    for l in range(int(cfg["n_layer"])):
        if sel is not None and l not in sel:
            continue
        p = f"blocks.{l}.ffn."
        layer = MoELayer(index=l, gate_weight=tensors[p + "gate.weight"], gate_bias=tensors.get(p + "gate.bias"),
                         top_k=k_top, tile=tile)
        for e in range(E):
            layer.experts.append(tuple(tensors[f"{p}experts.{e}.{q}.{b}"] for q in PROJ for b in ("w8", "sc")))
        if prepare and dev.type == "cuda":
            from smaulnative_amd.compute import get_backend
            get_backend("rocm").prepare_experts(layer.experts, d, h, tile)
        out.append(layer)
    return out


def load_into(module, layer: MoELayer):
    """Copy a loaded layer into a SwiFFN_MoE module's router and expert buffers (shapes checked)."""
    if len(module.experts) != len(layer.experts):
        raise RuntimeError(f"module has {len(module.experts)} experts, layer {len(layer.experts)}")
    with torch.no_grad():
        if tuple(module.gate.weight.shape) != tuple(layer.gate_weight.shape):
            raise RuntimeError(f"router shape {tuple(module.gate.weight.shape)} vs {tuple(layer.gate_weight.shape)}")
        module.gate.weight.copy_(layer.gate_weight)
        for ex, bufs in zip(module.experts, layer.experts):
            for dst, src in zip(ex.buffers6(), bufs):
                if tuple(dst.shape) != tuple(src.shape):
                    raise RuntimeError(f"expert buffer shape {tuple(dst.shape)} vs {tuple(src.shape)}")
                dst.copy_(src)
    return module
