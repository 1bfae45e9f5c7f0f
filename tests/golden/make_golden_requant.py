"""Writes tests/golden/golden_requant.npz from the reference's own FP8Linear.

Run in the build container only (the reference is not present on the GPU box):

    python tests/golden/make_golden_requant.py

Pins the weight-update path of kernel/fp8_tile.py:240-285: ``requant(update,
decay)`` (decode, scale by 1 - decay, subtract, quantize again) and
``fused_lion_requant(gw, st, lr, wd, b1, b2)`` (the Lion step folded into it),
whose codes depend on torch's fp32 elementwise rounding and on the quantizer's
argsort tie order.  The reference backend is set up as in make_golden.py (its
torch quantizer path).  Output: inputs and expected outputs only.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

from make_golden import _backend, _np as _view, ref_fp8  # noqa: E402


def _np(t):
    # a copy: requant and the Lion step rewrite their buffers in place, and a
    # numpy view of a CPU tensor would follow them
    return _view(t).copy()


def _module(in_f, out_f, tile, gen):
    m = ref_fp8.FP8Linear(in_f, out_f, tile=tile)
    with torch.no_grad():
        w8, sc = ref_fp8.quantize_tiles(torch.randn(out_f, in_f, generator=gen) * 0.05, tile)
        m.w8.copy_(w8)
        m.sc.copy_(sc)
    return m


def main():
    _backend()
    out = {}
    g = torch.Generator().manual_seed(77)
    # requant with an update and a decay; ragged last tile (100 = 3*32 + 4)
    for name, (in_f, out_f, tile, decay) in {"a": (100, 37, 32, 1e-3), "b": (130, 70, 64, 0.0),
                                             "c": (256, 96, 64, 0.05)}.items():
        m = _module(in_f, out_f, tile, g)
        upd = torch.randn(out_f, in_f, generator=g) * 0.02
        out[f"rq_{name}_w8"], out[f"rq_{name}_sc"] = _np(m.w8), _np(m.sc)
        out[f"rq_{name}_upd"] = _np(upd)
        out[f"rq_{name}_meta"] = np.array([in_f, out_f, tile, decay], dtype=np.float64)
        m.requant(upd, decay)
        out[f"rq_{name}_w8_out"], out[f"rq_{name}_sc_out"] = _np(m.w8), _np(m.sc)
    # requant without an update (decode + quantize again)
    m = _module(130, 33, 64, g)
    out["rq_none_w8"], out["rq_none_sc"] = _np(m.w8), _np(m.sc)
    m.requant(None, 0.0)
    out["rq_none_w8_out"], out["rq_none_sc_out"] = _np(m.w8), _np(m.sc)
    # Lion: bf16 gradient, fp32 momentum with a nonzero start
    lr, wd, b1, b2 = 2e-4, 0.01, 0.9, 0.99
    m = _module(128, 130, 32, g)
    gw = (torch.randn(130, 128, generator=g) * 1e-2).to(torch.bfloat16)
    st = torch.randn(130, 128, generator=g) * 1e-3
    out["lion_w8"], out["lion_sc"], out["lion_gw"], out["lion_st"] = _np(m.w8), _np(m.sc), _np(gw), _np(st)
    out["lion_meta"] = np.array([lr, wd, b1, b2], dtype=np.float64)
    m.fused_lion_requant(gw, st, lr, wd, b1, b2)
    out["lion_w8_out"], out["lion_sc_out"], out["lion_st_out"] = _np(m.w8), _np(m.sc), _np(st)
    path = os.path.join(HERE, "golden_requant.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, len(out), "arrays")


if __name__ == "__main__":
    main()
