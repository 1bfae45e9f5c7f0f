"""The tiled-E4M3 codebook shared by the quantizer, the decoder and the backend.

A code byte c decodes to sign(c) * magnitude(c) with e = (c >> 3) & 15 and
m = c & 7 (kernel/fp8_tile.py:39-48, kernel/fp8_cpu.cpp:16-26):
- e == 0: m * 2^-9 (subnormals; 0x00 is +0, 0x80 is -0);
- e == 15 and m == 7: 448 (so 0x7E and 0x7F are both 448, 0xFE and 0xFF -448;
  OCP E4M3FN would make 0x7F/0xFF NaN);
- otherwise (8 + m) * 2^(e - 10), i.e. (1 + m/8) * 2^(e - 7).
Every value is exact in fp32 and in bf16.

The encoder works on the codebook sorted by value: 255 midpoints between
neighbours, and the permutation from sorted position back to code.  The
permutation is torch.argsort's, computed on the CPU, because the codebook
has duplicate values and the stored codes depend on which duplicate the tie
order puts where (the reference builds its tables the same way,
kernel/fp8_tile.py:49-53; tests/golden pins the result).
"""
from __future__ import annotations

import functools

import torch

E4M3_MAX = 448.0


@functools.lru_cache(maxsize=None)
def _values_cpu() -> torch.Tensor:
    c = torch.arange(256, dtype=torch.int64)
    e, m = (c >> 3) & 15, c & 7
    mag = torch.where(e == 0, m.double() * 2.0 ** -9, (8 + m).double() * torch.pow(2.0, (e - 10).double()))
    mag = torch.where((e == 15) & (m == 7), torch.full_like(mag, E4M3_MAX), mag)
    sign = torch.where((c & 128) != 0, -1.0, 1.0).double()
    return (sign * mag).float()


@functools.lru_cache(maxsize=None)
def _tables_on(device: str, dtype: torch.dtype):
    v = _values_cpu()
    order = torch.argsort(v)
    ranked = v[order]
    mids = (ranked[:-1] + ranked[1:]) * 0.5
    return (v.to(device=device, dtype=dtype), order.to(device), mids.to(device=device, dtype=torch.float32),
            order.to(torch.uint8).to(device))


def values(device="cpu", dtype=torch.float32) -> torch.Tensor:
    """The 256 decoded values, indexed by code."""
    return _tables_on(str(torch.device(device)), dtype)[0]


def encode_tables(device="cpu"):
    """(order int64 [256], midpoints fp32 [255], order uint8 [256]) on ``device``."""
    t = _tables_on(str(torch.device(device)), torch.float32)
    return t[1], t[2], t[3]
