"""GPU parity of the tiled-FP8 linear's backward (training; not on the forward path).

fp8_backward_input (kernel/compute.py:145-153) against the oracle's
restatement of kernel/fp8_cpu.cpp:167-259, which the CPU tests pin bit-exact
to the reference's own kernel.  Bar: max relative difference 1e-5 -- the
GPU sums the output dimension in another fp32 order (the reference's own
test holds its kernel to 1e-5 against autograd, test_linear_fp8.py:186-199).
The module test runs FP8Linear forward + backward in training mode: the
input gradient, and the weight gradient accumulated in bf16 ``_gw`` in
64-row blocks (kernel/fp8_tile.py:172-197).
"""
import pytest
import torch

import oracle
from smaulnative_amd.compute import get_backend

pytestmark = pytest.mark.gpu
DEV = "cuda"


def rel_max(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-300))


@pytest.mark.parametrize("rows,in_f,out_f,tile", [(64, 128, 128, 64), (33, 70, 100, 64), (4096, 512, 1280, 64),
                                                  (50, 300, 130, 32), (17, 96, 200, 128), (1, 1024, 64, 64),
                                                  (0, 64, 64, 64)])
def test_backward_input_vs_oracle(rows, in_f, out_f, tile):
    print(f"case backward rows={rows} in_f={in_f} out_f={out_f} tile={tile}", flush=True)
    gen = torch.Generator().manual_seed(rows * 3 + in_f + out_f)
    g = torch.randn(rows, out_f, generator=gen)
    w, s = oracle.quantize_tiles(torch.randn(out_f, in_f, generator=gen) * 0.05, tile)
    dx = get_backend("rocm").fp8_backward_input(g.to(DEV), w.to(DEV), s.to(DEV), in_f, out_f, tile)
    assert dx.dtype == torch.float32 and tuple(dx.shape) == (rows, in_f)
    if rows == 0:
        return
    ref = oracle.fp8_backward_input(g, w, s, in_f, out_f, tile)
    assert rel_max(dx, ref) < 1e-5, rel_max(dx, ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fp8linear_training_step(dtype):
    from smaulnative_amd import FP8Linear
    torch.manual_seed(3)
    m = FP8Linear(192, 130, 64).to(DEV).train()
    x = torch.randn(2, 40, 192, device=DEV).to(dtype).requires_grad_(True)
    c = torch.randn(2, 40, 130, device=DEV)
    for step in range(2):  # the weight gradient accumulates across backward calls
        y = m(x)
        assert y.dtype == dtype
        (y.float() * c).sum().backward()
    # the module's output is in x's dtype, so the gradient reaching its backward
    # is c rounded to that dtype
    g = c.reshape(-1, 130).to(dtype).float().cpu()
    w, s = m.w8.cpu(), m.sc.cpu()
    gx = oracle.fp8_backward_input(g, w, s, 192, 130, 64).reshape(2, 40, 192)
    # two steps add the same gradient twice
    assert rel_max(x.grad.float(), (2 * gx).to(dtype).float()) < (1e-5 if dtype == torch.float32 else 8e-3)
    # _gw: per 64-row block, g^T x formed in fp32 and added to the bf16 buffer (rounded once per add)
    xr = x.detach().reshape(-1, 192).float().cpu()
    gw = torch.zeros(130, 192, dtype=torch.bfloat16)
    for _ in range(2):
        for o0 in range(0, 130, 64):
            gw[o0:o0 + 64].add_(g[:, o0:o0 + 64].t() @ xr)
    assert m._gw.dtype == torch.bfloat16 and tuple(m._gw.shape) == (130, 192)
    # the fp32 products are summed in another order on the device: a bf16
    # rounding may flip, and where the sum cancels the fp32 error bound (a few
    # units of 2^-24 of the sum of |terms|) can exceed one bf16 ulp of the result
    diff = (m._gw.cpu().float() - gw.float()).abs()
    ulp = gw.float().abs() * 2.0 ** -7
    terms = 2 * (g.abs().t() @ xr.abs())
    assert bool((diff <= 2 * ulp + terms * 2.0 ** -18).all())


@pytest.mark.parametrize("tile", [64, 128])
def test_backward_input_raw_codes(tile):
    """Every one of the 256 codes as stored (0x7F / 0xFF decode to +-448, NaN
    in OCP E4M3), scales spanning 2^-20..2^4, and a gradient with a wide
    dynamic range: the matrix-core form (tile a multiple of 64) splits g * s
    into three bf16 terms exactly and decodes the codes exactly."""
    rows, in_f, out_f = 200, 320, 512
    gen = torch.Generator().manual_seed(tile)
    w = torch.randint(0, 256, (out_f, in_f), generator=gen, dtype=torch.uint8)
    nt = (in_f + tile - 1) // tile
    s = torch.exp2(torch.randint(-20, 5, (out_f, nt), generator=gen).float()) * (1 + torch.rand(out_f, nt, generator=gen))
    g = torch.randn(rows, out_f, generator=gen) * torch.exp2(torch.randint(-30, 30, (rows, 1), generator=gen).float())
    dx = get_backend("rocm").fp8_backward_input(g.to(DEV), w.to(DEV), s.to(DEV), in_f, out_f, tile)
    ref = oracle.fp8_backward_input(g, w, s, in_f, out_f, tile)
    # per row: the rows differ by up to 2^60 in scale
    err = ((dx.cpu().double() - ref.double()).abs().amax(1) / ref.double().abs().amax(1).clamp_min(1e-300)).max()
    assert float(err) < 1e-5, float(err)


def test_backward_input_zero_sizes_abi():
    """in_f or out_f of 0 are accepted, as by the reference kernel
    (fp8_cpu.cpp:227-228): out_f == 0 is an empty sum (dx all zeros, g / w / s
    not read), in_f == 0 leaves nothing to write."""
    from smaulnative_amd import _lib
    lib = _lib.load()
    print("case backward_input zero sizes", flush=True)
    stream = torch.cuda.current_stream().cuda_stream
    dx = torch.full((3, 5), 7.0, device=DEV)
    _lib.check(lib.smaul_fp8_backward_input(None, None, None, dx.data_ptr(), 3, 5, 0, 64, stream), "out_f 0")
    _lib.check(lib.smaul_fp8_backward_input(None, None, None, None, 3, 0, 4, 64, stream), "in_f 0")
    torch.cuda.synchronize()
    assert torch.equal(dx.cpu(), torch.zeros(3, 5))
    assert lib.smaul_fp8_backward_input(None, None, None, dx.data_ptr(), 3, -1, 4, 64, stream) == _lib.SMAUL_ERR_INVALID
