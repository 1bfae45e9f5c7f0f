"""Tiled-E4M3 weights: the quantizer and the ``FP8Linear`` module.

Interface of the reference's kernel/fp8_tile.py (``TILE``, ``E4M3_MAX``,
``quantize_tiles``, ``decode_tile``, ``FP8Linear``, ``fp8_modules``), so model
code written against it runs unchanged.  The stored format is the
reference's: ``w8`` uint8 ``[out_f, in_f]`` codes and ``sc`` fp32
``[out_f, ceil(in_f / tile)]`` scales, one per output row and K tile, with no
fp32 master weight (kernel/fp8_tile.py:199-215).

``FP8Linear.forward(x)`` computes ``x @ decode(w8, sc).T`` through the
backend's ``fp8_forward`` and returns it in x's dtype (kernel/fp8_tile.py:
163-170, 237-239).  On the rocm backend bf16 activations go to the kernel as
they are (a bf16 value widened to fp32 is the same number).  The backward
takes the input gradient from the backend's ``fp8_backward_input`` and, in
training mode, adds the weight gradient to the module's bf16 ``_gw`` in
64-row blocks -- the storage the reference's optimizers read
(kernel/fp8_tile.py:172-197); there is no fp32 master weight.

``quantize_tiles`` gives the reference's codes and scales bit for bit: the
backend's device quantizer for HIP tensors (``fp8_quantize_tiles``), and the
same rules in torch ops for host tensors, where the backend contract's None
selects the torch path (kernel/compute.py:246-263).
"""
from __future__ import annotations

import math
import threading
import warnings

import torch
import torch.nn as nn

from smaulnative_amd import codebook
from smaulnative_amd.compute import get_backend

TILE = 64
E4M3_MAX = codebook.E4M3_MAX


def _quantize_torch(w32: torch.Tensor, tile: int):
    """The quantizer rules in torch ops on w32's device: (codes [out_f, nt*tile], sc, nonfinite)."""
    out_f, in_f = w32.shape
    nt = -(-in_f // tile)
    padded = torch.zeros(out_f, nt * tile, dtype=torch.float32, device=w32.device)
    padded[:, :in_f] = w32
    tiles = padded.view(out_f, nt, tile)
    finite = torch.isfinite(tiles)
    nonfinite = int((~finite).sum())
    amax = torch.where(finite, tiles.abs(), torch.zeros((), device=w32.device)).amax(dim=2)
    sc = (amax.clamp_min(1e-12) / E4M3_MAX).clamp_min(1e-12)
    n = torch.nan_to_num(tiles / sc.unsqueeze(-1), nan=0.0).clamp(-E4M3_MAX, E4M3_MAX)
    order, mids, _ = codebook.encode_tables(w32.device)
    codes = order[torch.bucketize(n, mids)]        # first midpoint >= n
    codes = torch.where(n == 0, torch.zeros_like(codes), codes)
    return codes.view(out_f, nt * tile).to(torch.uint8), sc, nonfinite


def quantize_tiles(w32, tile=TILE):
    """Per-(row, tile) scale amax/448 and nearest-codebook codes: (w8 [out_f, in_f], sc [out_f, nt])."""
    if tile <= 0:
        raise ValueError(f"tile must be > 0, got {tile}")
    if w32.dim() != 2:
        raise ValueError(f"w32 must be 2D [out_f, in_f], got dim={w32.dim()}")
    out_f, in_f = w32.shape
    if out_f <= 0 or in_f <= 0:
        raise ValueError(f"out_f/in_f must be positive, got {out_f}/{in_f}")
    with torch.no_grad():
        w = w32.detach().float().contiguous()
        res = get_backend().fp8_quantize_tiles(w, tile)
        codes, sc, nonfinite = res if res is not None else _quantize_torch(w, tile)
    if nonfinite:
        warnings.warn(f"quantize_tiles: {nonfinite} non-finite weight(s) saturated to finite E4M3",
                      RuntimeWarning, stacklevel=2)
    return codes[:, :in_f].contiguous(), sc


def decode_tile(w, s, o0, o1, t, tile=TILE, dtype=torch.float32):
    """Rows [o0, o1) of K tile t decoded: lut[codes] * scale, in ``dtype``."""
    lut = codebook.values(w.device, dtype)
    return lut[w[o0:o1, t * tile:(t + 1) * tile].long()] * s[o0:o1, t].to(dtype).unsqueeze(1)


def decode_block(w, s, o0, o1, in_f, tile=TILE, dtype=torch.float32):
    """Rows [o0, o1) of every K tile decoded: ``[o1-o0, in_f]`` in ``dtype``.

    Each value is the one product lut[code] * scale that decode_tile forms
    (kernel/fp8_tile.py:134-160), the ragged last tile included: the codes are
    padded to whole tiles so the scales broadcast over a [rows, nt, tile] view.
    """
    rows, nt = o1 - o0, -(-in_f // tile)
    lut = codebook.values(w.device, dtype)
    codes = w[o0:o1, :in_f].long()
    if nt * tile != in_f:
        codes = torch.nn.functional.pad(codes, (0, nt * tile - in_f))
    vals = lut[codes].view(rows, nt, tile) * s[o0:o1, :nt].to(dtype).unsqueeze(-1)
    return vals.view(rows, nt * tile)[:, :in_f]


GRAD_DTYPE = torch.bfloat16   # storage of the accumulated weight gradient (kernel/fp8_tile.py:26)
_GRAD_ROWS = 64               # weight-gradient rows added (and rounded) per step
_REQUANT_ELEMS = 1 << 24      # fp32 values decoded at once by requant (64 MB)
_GW_LOCK = threading.Lock()   # one for every module: it also keeps modules picklable


class _FP8Matmul(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w8, sc, in_f, out_f, tile, module):
        training = module is not None and module.training
        ctx.save_for_backward(x if training else None, w8, sc)
        ctx.dims = (in_f, out_f, tile, x.shape)
        ctx.module = module if training else None
        rows = x.reshape(-1, in_f)
        if not (rows.is_cuda and rows.dtype == torch.bfloat16):
            rows = rows.float()
        y = get_backend().fp8_forward(rows.contiguous(), w8, sc, in_f, out_f, tile)
        return y.reshape(*x.shape[:-1], out_f).to(x.dtype)

    @staticmethod
    def backward(ctx, grad):
        x, w8, sc = ctx.saved_tensors
        in_f, out_f, tile, xshape = ctx.dims
        g = grad.reshape(-1, out_f).float().contiguous()
        gx = None
        if ctx.needs_input_grad[0]:
            gx = get_backend().fp8_backward_input(g, w8, sc, in_f, out_f, tile).reshape(xshape)
        m = ctx.module
        if m is not None:
            # the weight gradient accumulates in the module's bf16 _gw, which the
            # reference's optimizers read and clear (kernel/fp8_tile.py:172-197):
            # each 64-row block of g^T x is formed in fp32 and rounded once
            xr = x.reshape(-1, in_f).float()
            with _GW_LOCK:  # backward passes on several threads add to one _gw
                if m._gw is None:
                    m._gw = torch.zeros(out_f, in_f, dtype=GRAD_DTYPE, device=g.device)
                elif m._gw.device != g.device:  # the module moved: keep what it accumulated
                    m._gw = m._gw.to(g.device)
                for o0 in range(0, out_f, _GRAD_ROWS):
                    o1 = min(o0 + _GRAD_ROWS, out_f)
                    m._gw[o0:o1].add_(g[:, o0:o1].t() @ xr)
        return gx, None, None, None, None, None, None


class FP8Linear(nn.Module):
    """Linear layer over tiled-E4M3 weights: buffers ``w8`` / ``sc``, optional fp32 ``bias``."""

    def __init__(self, in_f, out_f, tile=TILE, bias=False):
        super().__init__()
        if in_f <= 0 or out_f <= 0:
            raise ValueError(f"in_f/out_f must be positive, got {in_f}/{out_f}")
        if tile <= 0:
            raise ValueError(f"tile must be > 0, got {tile}")
        self.in_f, self.out_f, self.tile = in_f, out_f, tile
        # nn.Linear's default weight distribution, U(-1/sqrt(in_f), 1/sqrt(in_f)), quantized
        bound = 1.0 / math.sqrt(in_f)
        w8, sc = quantize_tiles(torch.empty(out_f, in_f).uniform_(-bound, bound), tile)
        self.register_buffer("w8", w8)
        self.register_buffer("sc", sc)
        self.bias = nn.Parameter(torch.zeros(out_f)) if bias else None
        self._gw = None  # accumulated weight gradient (training), GRAD_DTYPE [out_f, in_f]

    @classmethod
    def from_float(cls, lin, tile=TILE):
        """An FP8Linear holding ``lin``'s weight (and bias) quantized."""
        m = cls(lin.in_features, lin.out_features, tile, lin.bias is not None)
        with torch.no_grad():
            w8, sc = quantize_tiles(lin.weight.detach().float(), tile)
            m.w8.copy_(w8)
            m.sc.copy_(sc)
            if lin.bias is not None:
                m.bias.copy_(lin.bias.detach())
        return m

    def forward(self, x):
        y = _FP8Matmul.apply(x, self.w8, self.sc, self.in_f, self.out_f, self.tile, self)
        return y if self.bias is None else y + self.bias

    def extra_repr(self):
        return f"in_f={self.in_f}, out_f={self.out_f}, tile={self.tile}, bias={self.bias is not None}"

    # -- weight updates: decode, apply, quantize again (kernel/fp8_tile.py:240-285) --
    # Quantization is per (row, tile), so rows may be processed in any grouping
    # with the same codes; the groups here only bound the fp32 temporary.
    def _row_groups(self):
        step = max(1, _REQUANT_ELEMS // max(1, self.in_f))
        for o0 in range(0, self.out_f, step):
            yield o0, min(o0 + step, self.out_f)

    @torch.no_grad()
    def _requant_rows(self, o0, o1, update, decay):
        w = decode_block(self.w8, self.sc, o0, o1, self.in_f, self.tile)
        if decay:
            w.mul_(1 - decay)
        if update is not None:
            w.sub_(update.to(w.dtype))
        codes, scales = quantize_tiles(w, self.tile)
        self.w8[o0:o1].copy_(codes)
        self.sc[o0:o1].copy_(scales)

    @torch.no_grad()
    def requant(self, update=None, decay=0.0):
        """W <- quantize(decode(W) * (1 - decay) - update) in place; clears ``_gw``.

        ``update`` is ``[out_f, in_f]`` (any float dtype) or None.  HIP buffers
        are decoded and quantized on the device.
        """
        if update is not None and (update.dim() != 2 or tuple(update.shape) != (self.out_f, self.in_f)):
            raise ValueError(f"requant update must be [{self.out_f}, {self.in_f}], got {tuple(update.shape)} "
                             "(a transposed [in_f, out_f] update is the usual mistake)")
        for o0, o1 in self._row_groups():
            self._requant_rows(o0, o1, None if update is None else update[o0:o1], decay)
        self._gw = None

    @torch.no_grad()
    def fused_lion_requant(self, gw, st, lr, wd, b1, b2):
        """One Lion step folded into requant: the update sign(b1*m + (1-b1)*g) * lr
        with decay lr * wd, the fp32 momentum ``st`` advanced in place to
        b2*m + (1-b2)*g; the same elementwise formulas as the reference
        (kernel/fp8_tile.py:266-282), so codes and momentum match it bit for bit.
        Clears ``_gw``."""
        for o0, o1 in self._row_groups():
            g = gw[o0:o1].float()
            m = st[o0:o1]
            step = (m * b1 + g * (1.0 - b1)).sign() * lr
            m.mul_(b2).add_(g, alpha=1.0 - b2)
            self._requant_rows(o0, o1, step, lr * wd)
        self._gw = None

    def err_stats(self):
        """{"amax_fp8": largest |decoded weight|, "mean_scale": mean of the scales}."""
        with torch.no_grad():
            amax = 0.0
            for o0, o1 in self._row_groups():
                amax = max(amax, float(decode_block(self.w8, self.sc, o0, o1, self.in_f, self.tile).abs().amax()))
            return {"amax_fp8": amax, "mean_scale": float(self.sc.double().mean())}


def fp8_modules(model):
    """(name, module) of every FP8Linear in ``model``."""
    return [(n, m) for n, m in model.named_modules() if isinstance(m, FP8Linear)]
