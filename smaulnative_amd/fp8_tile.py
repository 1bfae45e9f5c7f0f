"""Tiled-E4M3 storage and ``FP8Linear``, the interface of the reference's kernel/fp8_tile.py.

Storage is unchanged (fp8_tile.py:199-215): buffers ``w8`` uint8
``[out_f, in_f]`` and ``sc`` fp32 ``[out_f, ceil(in_f/tile)]``; no fp32
master weight.  ``FP8Linear.forward`` keeps the reference signature and
dtype behaviour (fp8_tile.py:163-170,237-239): the GEMM accumulates in fp32
and the result is cast to ``x.dtype``.  The GEMM runs through
``get_backend().fp8_forward``; bf16 activations are handed over as bf16 (the
rocm backend feeds them to bf16 MFMA unchanged, which is exact: a bf16 value
widened to fp32 is the same number).

The quantizer is the reference's torch path (fp8_tile.py:82-119), used for
weight preparation only (module construction, ``from_float``); the backend's
``fp8_quantize_tiles`` returns ``None`` to select it, as the backend contract
allows (compute.py:246-263).
"""
from __future__ import annotations

import math
import threading
import warnings

import torch
import torch.nn as nn

from smaulnative_amd.compute import get_backend

TILE = 64
_OB = 64
E4M3_MAX = 448.0

_LUT_CACHE: dict = {}
_LUT_MAX_ENTRIES = 32


def _codebook_values() -> torch.Tensor:
    """fp8_tile.py:39-48: e=(c>>3)&15, m=c&7; 0x7F/0xFF -> +-448; e=0 -> +-m*2^-9."""
    v = torch.empty(256, dtype=torch.float32)
    for c in range(256):
        e, m = (c >> 3) & 15, c & 7
        s = -1.0 if c & 128 else 1.0
        if e == 15 and m == 7:
            v[c] = s * 448.0
        elif e == 0:
            v[c] = s * m * 2.0 ** -9
        else:
            v[c] = s * (1 + m / 8.0) * 2.0 ** (e - 7)
    return v


def _tables(device, dtype=torch.float32):
    """(lut, order, sorted values, midpoints), LRU-cached per (device, dtype) (fp8_tile.py:31-57)."""
    key = (str(device), str(dtype))
    hit = _LUT_CACHE.get(key)
    if hit is not None:
        _LUT_CACHE.pop(key)
        _LUT_CACHE[key] = hit
        return hit
    v = _codebook_values()
    order = torch.argsort(v)
    sval = v[order]
    out = (v.to(device=device, dtype=dtype), order.to(device),
           sval.to(device=device, dtype=dtype),
           ((sval[:-1] + sval[1:]) * 0.5).to(device=device, dtype=dtype))
    if len(_LUT_CACHE) >= _LUT_MAX_ENTRIES:
        _LUT_CACHE.pop(next(iter(_LUT_CACHE)))
    _LUT_CACHE[key] = out
    return out


def _lut(device, dtype=torch.float32):
    return _tables(device, dtype)[0]


def quantize_tiles(w32, tile=TILE):
    """Per-(row, tile) absmax/448 scale and nearest-codebook codes (fp8_tile.py:82-119)."""
    if tile <= 0:
        raise ValueError(f"tile must be > 0, got {tile}")
    if w32.dim() != 2:
        raise ValueError(f"w32 must be 2D [out_f, in_f], got dim={w32.dim()}")
    out_f, in_f = w32.shape
    if out_f <= 0 or in_f <= 0:
        raise ValueError(f"out_f/in_f must be positive, got {out_f}/{in_f}")
    with torch.no_grad():
        w32 = w32.float().contiguous()
        nt = (in_f + tile - 1) // tile
        native = get_backend().fp8_quantize_tiles(w32, tile)
        if native is not None:
            codes, sc, nonfinite = native
        else:
            pad = nt * tile - in_f
            if pad:
                w32 = torch.cat([w32, torch.zeros(out_f, pad, dtype=w32.dtype, device=w32.device)], 1)
            nonfinite = int((~torch.isfinite(w32)).sum())
            _, order, _, bounds = _tables(w32.device, torch.float32)
            blk = w32.reshape(out_f, nt, tile)
            amax = torch.where(torch.isfinite(blk), blk.abs(), 0.0).amax(dim=2).clamp_min(1e-12)
            sc = (amax / E4M3_MAX).clamp_min(1e-12)
            n = torch.nan_to_num(blk / sc[..., None], nan=0.0).clamp(-E4M3_MAX, E4M3_MAX)
            nf = n.reshape(-1)
            codes = order[torch.bucketize(nf, bounds).clamp(0, 255)].reshape(out_f, nt * tile)
            codes.reshape(-1)[nf == 0] = 0
        if nonfinite:
            warnings.warn(f"quantize_tiles: {nonfinite} non-finite weight(s) saturated to finite E4M3",
                          RuntimeWarning, stacklevel=2)
        return codes[:, :in_f].contiguous().to(torch.uint8), sc


def decode_tile(w, s, o0, o1, t, tile=TILE, dtype=torch.float32):
    """Rows [o0:o1] of tile t decoded to ``dtype`` (fp8_tile.py:121-131)."""
    lut = _lut(w.device, dtype)
    blk = w[o0:o1, t * tile:(t + 1) * tile].long()
    return lut[blk] * s[o0:o1, t].to(dtype)[:, None]


class _Fn(torch.autograd.Function):
    """fp8_tile.py:162-170 forward.  Backward asks the backend (the rocm backend raises)."""

    @staticmethod
    def forward(ctx, x, w, s, in_f, out_f, tile, mod):
        ctx.save_for_backward(w, s)
        ctx.in_f, ctx.out_f, ctx.tile, ctx.xshape = in_f, out_f, tile, x.shape
        x2 = x.reshape(-1, in_f)
        if not (x2.dtype == torch.bfloat16 and x2.is_cuda):
            x2 = x2.float()
        x2 = x2.contiguous()
        y = get_backend().fp8_forward(x2, w, s, in_f, out_f, tile)
        return y.reshape(*x.shape[:-1], out_f).to(x.dtype)

    @staticmethod
    def backward(ctx, g):
        w, s = ctx.saved_tensors
        g2 = g.reshape(-1, ctx.out_f).float().contiguous()
        gx = get_backend().fp8_backward_input(g2, w, s, ctx.in_f, ctx.out_f, ctx.tile)
        return gx.reshape(ctx.xshape), None, None, None, None, None, None


class FP8Linear(nn.Module):
    """Tiled-E4M3 linear layer with the reference's buffers and forward signature."""

    def __init__(self, in_f, out_f, tile=TILE, bias=False):
        super().__init__()
        if in_f <= 0 or out_f <= 0:
            raise ValueError(f"in_f/out_f must be positive, got {in_f}/{out_f}")
        if tile <= 0:
            raise ValueError(f"tile must be > 0, got {tile}")
        self.in_f, self.out_f, self.tile = in_f, out_f, tile
        self._gw_lock = threading.Lock()
        w0 = torch.empty(out_f, in_f, dtype=torch.float32)
        nn.init.kaiming_uniform_(w0, a=math.sqrt(5))
        wq, sq = quantize_tiles(w0, tile)
        self.register_buffer("w8", wq)
        self.register_buffer("sc", sq)
        self.bias = nn.Parameter(torch.zeros(out_f)) if bias else None
        self._gw = None

    def __getstate__(self):
        state = self.__dict__.copy()
        state.pop("_gw_lock", None)
        return state

    def __setstate__(self, state):
        self.__dict__.update(state)
        self._gw_lock = threading.Lock()

    @classmethod
    def from_float(cls, lin, tile=TILE):
        m = cls(lin.in_features, lin.out_features, tile, lin.bias is not None)
        wq, sq = quantize_tiles(lin.weight.detach().float(), tile)
        m.w8.copy_(wq)
        m.sc.copy_(sq)
        if lin.bias is not None and m.bias is not None:
            with torch.no_grad():
                m.bias.copy_(lin.bias.detach())
        return m

    def forward(self, x):
        out = _Fn.apply(x, self.w8, self.sc, self.in_f, self.out_f, self.tile, self)
        return out if self.bias is None else out + self.bias


def fp8_modules(model):
    return [(n, m) for n, m in model.named_modules() if isinstance(m, FP8Linear)]
