"""GPU parity of the tiled-E4M3 quantizer (the backend's fp8_quantize_tiles).

Bar: codes, scales and the non-finite count bit-identical to the reference
quantizer -- its golden vectors (the 12 special-value cases of
tests/test_linear_fp8.py:484-510 x tiles 32/64/128, written from the
reference by tests/golden/make_golden.py) and the oracle's torch path
(kernel/fp8_tile.py:100-113), which the CPU tests pin to those vectors.
"""
import os
import warnings

import numpy as np
import pytest
import torch

import oracle
from smaulnative_amd.compute import get_backend
from smaulnative_amd.fp8_tile import decode_tile, quantize_tiles

pytestmark = pytest.mark.gpu

DEV = "cuda"
GOLD = os.path.join(os.path.dirname(__file__), "golden", "golden_fp8_moe.npz")
QCASES = ["uniform", "tiny", "huge", "zeros", "half_zero", "codebook", "midpoints", "saturating",
          "subnormal", "odd_shape", "padded_tile", "nonfinite"]


@pytest.mark.parametrize("tile", [32, 64, 128])
def test_device_quantizer_golden(tile):
    g = np.load(GOLD)
    be = get_backend("rocm")
    for name in QCASES:
        w = torch.from_numpy(np.array(g[f"q_{name}_w"]))
        print(f"case quant {name} {tuple(w.shape)} tile={tile}", flush=True)
        codes, sc, bad = be.fp8_quantize_tiles(w.to(DEV), tile)
        in_f = w.shape[1]
        assert codes.shape[1] == -(-in_f // tile) * tile
        assert bool((codes[:, in_f:] == 0).all())                     # the padding of the last tile
        assert np.array_equal(codes[:, :in_f].cpu().numpy(), g[f"q_{name}_t{tile}_codes"])
        assert np.array_equal(sc.cpu().numpy().view(np.uint32), g[f"q_{name}_t{tile}_sc"].view(np.uint32))
        assert bad == int((~torch.isfinite(w)).sum())


@pytest.mark.parametrize("out_f,in_f,tile", [(2560, 1024, 64), (77, 333, 32), (64, 200, 48), (33, 1000, 100),
                                             (16, 640, 128), (9, 70, 1), (40, 96, 8), (5, 300, 256)])
def test_device_quantizer_vs_oracle(out_f, in_f, tile):
    print(f"case quant random {out_f}x{in_f} tile={tile}", flush=True)
    gen = torch.Generator().manual_seed(out_f * 31 + in_f + tile)
    w = torch.randn(out_f, in_f, generator=gen) * 0.02
    w[torch.rand(out_f, in_f, generator=gen) < 0.01] = 0.0
    ref_c, ref_s = oracle.quantize_tiles(w, tile)
    c, s = quantize_tiles(w.to(DEV), tile)          # the product entry, device path
    assert c.is_cuda and c.dtype == torch.uint8 and tuple(c.shape) == (out_f, in_f)
    assert torch.equal(c.cpu(), ref_c)
    assert torch.equal(s.cpu(), ref_s)
    # decoding on the device gives the oracle's values
    t = min(1, s.shape[1] - 1)
    assert torch.equal(decode_tile(c, s, 0, out_f, t, tile).cpu(), oracle.decode_tile(ref_c, ref_s, 0, out_f, t, tile))


def test_device_quantizer_warns_on_nonfinite():
    w = torch.randn(8, 64)
    w[0, 0], w[1, 1] = float("nan"), float("inf")
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        c, s = quantize_tiles(w.to(DEV), 64)
    assert any("2 non-finite" in str(r.message) for r in rec)
    ref_c, ref_s = oracle.quantize_tiles(w, 64)
    assert torch.equal(c.cpu(), ref_c) and torch.equal(s.cpu(), ref_s)
