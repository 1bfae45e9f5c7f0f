"""GPU parity over seeded sweeps of shapes: moe_forward, fp8_forward and the
dense SwiFFN against the oracle.

Each case draws T (1 .. 3000, around the 64-token decode limit and the 128-row
tile edges), d and h (multiples of 64), E (1 .. 16), top-k (1 .. min(E, 4)),
the activation dtype (bf16 or fp32), the scale tile (32 for fp32, 64, 128) and,
for one case in five, a router bias that sends every token to expert 0.  The
cases are fixed by the seed, so a failure names a reproducible shape.  Bars as
in test_gpu_parity: routing and counts bit-exact; rel-L2 <= 2e-3 with bf16
activations, <= 1e-5 with fp32 (fp8_forward: max-relative 2e-6 / 1e-5).
"""
import random

import pytest
import torch

import oracle
from test_gpu_parity import be, gpu_moe, make_moe, rel_l2, rel_max

pytestmark = pytest.mark.gpu

T_CHOICES = [1, 2, 7, 16, 33, 63, 64, 65, 100, 129, 255, 300, 511, 700, 1023, 1500, 2049, 3000]


def _cases(seed, n):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        T = rng.choice(T_CHOICES)
        d = 64 * rng.randint(1, 16)
        h = 64 * rng.randint(1, 24)
        E = rng.randint(1, 16)
        k = rng.randint(1, min(E, 4))
        f32 = rng.random() < 0.3
        tile = rng.choice([64, 64, 64, 128, 32]) if f32 else rng.choice([64, 64, 128])
        while T * k * d * h > 1.5e10:  # keeps each oracle call to about a second
            if h > 128:
                h = (h // 2) - (h // 2) % 64
            elif d > 128:
                d = (d // 2) - (d // 2) % 64
            else:
                T //= 2
        if d % tile or h % tile:
            tile = 64
        skew = rng.random() < 0.2 and E > 1
        out.append((T, d, h, E, k, f32, tile, skew))
    return out


@pytest.mark.parametrize("case", _cases(20261202, 48), ids=lambda c: "T{}-d{}-h{}-E{}-k{}-{}-t{}{}".format(
    c[0], c[1], c[2], c[3], c[4], "f32" if c[5] else "bf16", c[6], "-skew" if c[7] else ""))
def test_moe_shape_sweep(case):
    T, d, h, E, k, f32, tile, skew = case
    dtype = torch.float32 if f32 else torch.bfloat16
    print(f"case sweep T={T} d={d} h={h} E={E} k={k} {dtype} tile={tile} skew={skew}", flush=True)
    x, gw, gb, experts = make_moe(T * 31 + d + E, T, d, h, E, k, dtype, tile=tile,
                                  skew=(9.0, [], 0.0) if skew else None)
    ref = oracle.moe_forward(x, gw, gb, experts, k, tile)
    out, prob, topi, counts = gpu_moe(x, gw, gb, experts, k, tile)
    assert torch.equal(topi.reshape(-1, k), ref.topi.reshape(-1, k))
    assert counts.tolist() == ref.counts
    if skew:
        assert ref.counts[0] == T
    err = rel_l2(out.float(), ref.out.float())
    print(f"rel_l2={err:.3e}")
    assert err < (2e-3 if dtype == torch.bfloat16 else 1e-5)


def _dense_cases(seed, n):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        rows = rng.choice([1, 3, 64, 65, 127, 300, 513, 1024, 1025, 2500, 4096])
        in_f = rng.choice([rng.randint(1, 300), 64 * rng.randint(1, 32)])
        out_f = rng.choice([rng.randint(1, 300), 64 * rng.randint(1, 40)])
        f32 = rng.random() < 0.5
        tile = rng.choice([64, 64, 64, 128, 32])
        out.append((rows, in_f, out_f, f32, tile))
    return out


@pytest.mark.parametrize("case", _dense_cases(1202, 32), ids=lambda c: "r{}-i{}-o{}-{}-t{}".format(
    c[0], c[1], c[2], "f32" if c[3] else "bf16", c[4]))
def test_fp8_forward_shape_sweep(case):
    """fp8_forward (FP8Linear's GEMM) over ragged and tile-aligned shapes:
    whichever kernel the shape selects (LDS-DMA tiles sized to the grid, the
    in-LDS or workspace fp32 split, the register-staged kernel), every row
    against the oracle at the bar of its input dtype."""
    rows, in_f, out_f, f32, tile = case
    print(f"case sweep fp8_forward rows={rows} in_f={in_f} out_f={out_f} f32={f32} tile={tile}", flush=True)
    gen = torch.Generator().manual_seed(rows * 3 + in_f * 5 + out_f * 7 + tile)
    x = torch.randn(rows, in_f, generator=gen)
    if not f32:
        x = x.to(torch.bfloat16)
    w, s = oracle.quantize_tiles(torch.randn(out_f, in_f, generator=gen) * 0.02, tile)
    y = be().fp8_forward(x.to("cuda"), w.to("cuda"), s.to("cuda"), in_f, out_f, tile).cpu()
    ref = oracle.fp8_forward(x.float(), w, s, in_f, out_f, tile)
    assert y.shape == (rows, out_f) and torch.isfinite(y).all()
    assert rel_max(y, ref) < (1e-5 if f32 else 2e-6), rel_max(y, ref)


@pytest.mark.parametrize("case", [c for c in _dense_cases(1203, 24) if c[1] % 64 == 0 and c[2] % 64 == 0][:12],
                         ids=lambda c: "r{}-d{}-h{}-{}-t{}".format(c[0], c[1], c[2], "f32" if c[3] else "bf16", c[4]))
def test_swiffn_shape_sweep(case):
    """The dense SwiGLU FFN (gate+up in one launch, then down) over a sweep of
    shapes, against the oracle's three FP8Linear calls."""
    rows, d, h, f32, tile = case
    if d % tile or h % tile:
        tile = 64
    dtype = torch.float32 if f32 else torch.bfloat16
    print(f"case sweep swiffn rows={rows} d={d} h={h} {dtype} tile={tile}", flush=True)
    gen = torch.Generator().manual_seed(rows * 11 + d + h * 3)
    x = torch.randn(rows, d, generator=gen).to(dtype)
    ex = oracle.make_expert(d, h, gen, tile)
    bufs = tuple(t.to("cuda") for t in (ex.gate_w, ex.gate_s, ex.up_w, ex.up_s, ex.down_w, ex.down_s))
    y = be().swiffn_forward(x.to("cuda"), bufs, tile).cpu()
    ref = oracle.swiffn_forward(x, ex, tile)
    assert y.dtype == dtype
    err = rel_l2(y.float(), ref.float())
    print(f"rel_l2={err:.3e}")
    assert err < (2e-3 if dtype == torch.bfloat16 else 1e-5)
