"""``SwiFFN`` and ``SwiFFN_MoE`` with the reference's interface (model.py:282-290, 506-606).

``SwiFFN_MoE.forward(x)`` keeps the reference signature, output dtype and the
diagnostic attributes read by training logs and retention reports:
``last_prob``, ``last_topi``, ``last_executed``, ``expert_token_counts``,
``routing_stats()``, ``reset_routing_stats()``, ``balance_loss(prob)``.

The whole layer (router, dispatch, the expert SwiGLU GEMMs, combine) is one
call to the backend's ``moe_forward``; the per-expert Python loop with a host
sync per expert (model.py:574-582) is gone.  When autograd must record the
layer (grad mode on and the input or a parameter requiring grad, in train and
eval mode alike) it runs as device torch ops around the experts' FP8Linear
kernels instead, so gradients reach the input, the router and the experts'
weight gradients (``_forward_train``).  ``expert_token_counts`` and
``last_executed`` are materialised from the device counts only when read, so
a decode step does not force a device->host sync per layer.

Only the plain architecture's dense SwiGLU experts are on this path; the rawr
(sparse) experts are not (model.py:528-534).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from smaulnative_amd.compute import get_backend
from smaulnative_amd.fp8_tile import FP8Linear


@dataclass
class MoEConfig:
    """The LinearConfig fields (model.py:18-40) the MoE layer reads.

    A reference ``LinearConfig`` instance works in its place (same names).
    """
    d_model: int = 512
    ffn_mult: float = 2.5
    tile: int = 64
    num_experts: int = 1
    num_experts_per_tok: int = 1
    precision: str = "fp8"
    architecture: str = "plain"

    def __post_init__(self):
        for name in ("d_model", "tile", "num_experts", "num_experts_per_tok"):
            v = getattr(self, name)
            if not isinstance(v, int) or v <= 0:
                raise ValueError(f"{name} must be a positive int, got {v!r}")
        if self.num_experts_per_tok > self.num_experts:
            raise ValueError(f"num_experts_per_tok ({self.num_experts_per_tok}) > "
                             f"num_experts ({self.num_experts})")


def _needs_grad(module: nn.Module, x: torch.Tensor) -> bool:
    """Whether the forward must record autograd: grad mode on and x or a
    parameter of ``module`` requiring grad, in train and eval mode alike (as
    with the reference's autograd function, kernel/fp8_tile.py:162-170; the
    module's training flag only decides whether FP8Linear accumulates ``_gw``).
    The fused device entries keep no activations, so they run only otherwise."""
    if not torch.is_grad_enabled():
        return False
    return x.requires_grad or any(p.requires_grad for p in module.parameters())


class SwiFFN(nn.Module):
    """model.py:282-290: down((silu(gate(x).float()) * up(x).float()).to(x.dtype))."""

    def __init__(self, cfg):
        super().__init__()
        if cfg.precision != "fp8":
            raise ValueError("the rocm path implements precision='fp8' experts only")
        h = int(cfg.d_model * cfg.ffn_mult)
        self.gate = FP8Linear(cfg.d_model, h, cfg.tile)
        self.up = FP8Linear(cfg.d_model, h, cfg.tile)
        self.down = FP8Linear(h, cfg.d_model, cfg.tile)

    def forward(self, x):
        be = get_backend()
        if hasattr(be, "swiffn_forward") and not _needs_grad(self, x):
            xf = x if x.is_floating_point() else x.float()
            return be.swiffn_forward(xf, self.buffers6(), self.gate.tile)
        odt = x.dtype if x.is_floating_point() else torch.float32
        return self.down((F.silu(self.gate(x).float()) * self.up(x).float()).to(odt))

    def buffers6(self):
        return (self.gate.w8, self.gate.sc, self.up.w8, self.up.sc, self.down.w8, self.down.sc)


class SwiFFN_MoE(nn.Module):
    """Top-k routed mixture of SwiFFN experts (model.py:506-606)."""

    def __init__(self, cfg, rawr_graph=None):
        super().__init__()
        if cfg.num_experts < 1 or cfg.num_experts_per_tok < 1:
            raise ValueError("num_experts and num_experts_per_tok must be >= 1")
        if cfg.num_experts_per_tok > cfg.num_experts:
            raise ValueError(
                f"num_experts_per_tok ({cfg.num_experts_per_tok}) > num_experts ({cfg.num_experts})")
        if getattr(cfg, "architecture", "plain") != "plain":
            raise ValueError("the rocm MoE path implements architecture='plain' (SwiFFN experts) only")
        self.top_k = cfg.num_experts_per_tok
        self.num_experts = cfg.num_experts
        self.architecture = "plain"
        self.tile = cfg.tile
        self.experts = nn.ModuleList([SwiFFN(cfg) for _ in range(cfg.num_experts)])
        self.gate = nn.Linear(cfg.d_model, cfg.num_experts, bias=False)
        self.last_prob = None
        self.last_topi = None
        self._counts_dev = None
        self._counts_host = [0] * cfg.num_experts

    # -- diagnostics (model.py:538-543,583-584,587-606), materialised lazily --
    @property
    def expert_token_counts(self):
        if self._counts_dev is not None:
            self._counts_host = [int(c) for c in self._counts_dev.tolist()]
            self._counts_dev = None
        return self._counts_host

    @expert_token_counts.setter
    def expert_token_counts(self, value):
        self._counts_dev = None
        self._counts_host = list(value)

    @property
    def last_executed(self):
        return [c > 0 for c in self.expert_token_counts]

    @last_executed.setter
    def last_executed(self, value):
        # kept for interface compatibility; executed is derived from counts
        pass

    def balance_loss(self, prob: torch.Tensor) -> torch.Tensor:
        """Switch-style load-balancing aux loss (model.py:545-555)."""
        density = prob.mean(0)
        return (density * density * self.num_experts).sum()

    def forward(self, x):
        be = get_backend()
        if not hasattr(be, "moe_forward"):
            raise RuntimeError(f"compute backend {be.name!r} has no moe_forward entry")
        if _needs_grad(self, x):
            return self._forward_train(x)
        experts = [ex.buffers6() for ex in self.experts]
        out, prob, topi, counts = be.moe_forward(x, self.gate.weight, self.gate.bias, experts,
                                                 self.top_k, self.tile)
        self.last_prob = prob
        self.last_topi = topi
        self._counts_dev = counts
        return out

    def _forward_train(self, x):
        """The layer with autograd, for training.

        The router softmax, top-k and renormalisation of model.py:557-570 as
        torch ops on the device (gradient reaches the router through the
        selected probabilities only, as in the reference); each expert's rows
        gathered and run through its SwiFFN, whose FP8Linear modules compute
        the forward and the input gradient with the backend's kernels and
        accumulate their weight gradients in ``_gw``; the weighted outputs added
        back token by token in ascending expert order (model.py:571-585).  The
        fused moe_forward path has no backward, so training runs this one.
        """
        d = x.shape[-1]
        lead = x.shape[:-1]
        xs = x.reshape(-1, d)
        prob = torch.softmax(self.gate(xs.float()), -1)
        # kept with x's leading dimensions, as the reference's are (model.py:558-565)
        self.last_prob = prob.view(*lead, self.num_experts)
        topv, topi = torch.topk(prob, self.top_k, -1)
        self.last_topi = topi.detach().view(*lead, self.top_k)
        total = topv.sum(-1, keepdim=True)
        topv = torch.where(total < 1e-6, torch.full_like(topv, 1.0 / self.top_k), topv / total.clamp_min(1e-9))
        out = torch.zeros(xs.shape, dtype=torch.float32, device=xs.device)
        counts = []
        for e, expert in enumerate(self.experts):
            weight = torch.where(topi == e, topv, torch.zeros_like(topv)).sum(-1)
            rows = torch.nonzero(weight > 0).squeeze(-1)
            counts.append(int(rows.numel()))
            if counts[-1]:
                y = expert(xs.index_select(0, rows)).float() * weight.index_select(0, rows).unsqueeze(-1)
                out = out.index_add(0, rows, y)
        self.expert_token_counts = counts
        return out.view(x.shape).to(x.dtype if x.is_floating_point() else torch.float32)

    def routing_stats(self) -> dict:
        counts = list(self.expert_token_counts)
        total = sum(counts)
        usage = [(c / total) if total else 0.0 for c in counts]
        return {
            "num_experts": self.num_experts,
            "top_k": self.top_k,
            "token_counts": counts,
            "usage_frac": usage,
            "executed": [c > 0 for c in counts],
            "inactive_experts": sum(1 for c in counts if c == 0),
            "max_usage_frac": max(usage) if usage else 0.0,
        }

    def reset_routing_stats(self) -> None:
        self.last_prob = None
        self.last_topi = None
        self._counts_dev = None
        self._counts_host = [0] * self.num_experts
