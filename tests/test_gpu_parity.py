"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Bars:
- routing indices, permutation and counts bit-exact;
- outputs within rel-L2 <= 2e-3 of the reference CPU path with bf16
  activations (the same bf16 x fed to both sides) and fp32 accumulation.
The GEMM itself is held much tighter: the MFMA products x*lut are exact in
fp32 and the scale is applied per tile in fp32, so only accumulation order
differs from the reference's sequential sum.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from smaulnative_amd.compute import get_backend

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden", "golden_fp8_moe.npz")
DEV = "cuda"


def rel_l2(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


def rel_max(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-300))


def be():
    b = get_backend("rocm")
    assert b.has_native, "libsmaul_rocm.so must be built (no fallback exists)"
    return b


def to_dev_experts(experts):
    return [tuple(t.to(DEV) for t in (ex.gate_w, ex.gate_s, ex.up_w, ex.up_s, ex.down_w, ex.down_s))
            for ex in experts]


def make_moe(seed, T, d, h, E, k, dtype=torch.bfloat16, bias_std=0.5, tile=64, skew=None):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(T, d, generator=gen)
    gw = torch.randn(E, d, generator=gen) * 0.02
    gb = torch.randn(E, generator=gen) * bias_std if bias_std else None
    if skew is not None:
        gb = torch.zeros(E)
        gb[0] = skew[0]
        for e in skew[1]:
            gb[e] = -skew[2]
    experts = [oracle.make_expert(d, h, gen, tile) for _ in range(E)]
    return x.to(dtype), gw, gb, experts


def gpu_moe(x, gw, gb, experts, k, tile=64):
    out, prob, topi, counts = be().moe_forward(x.to(DEV), gw.to(DEV), None if gb is None else gb.to(DEV),
                                               to_dev_experts(experts), k, tile)
    torch.cuda.synchronize()
    return out.cpu(), prob.cpu(), topi.cpu(), counts.cpu()


def route_margin(prob, topi, k):
    """Gap between the k-th selected and the best unselected probability."""
    p = prob.reshape(-1, prob.shape[-1]).double()
    sel = torch.zeros_like(p, dtype=torch.bool)
    sel.scatter_(1, topi.reshape(-1, k), True)
    kth = p.masked_fill(~sel, float("inf")).min(1).values
    rest = p.masked_fill(sel, float("-inf")).max(1).values
    return kth - rest


# --------------------------------------------------------------------------
# dense FP8 linear
# --------------------------------------------------------------------------
def test_fp8_linear_golden_fp32_inputs():
    g = np.load(GOLD)
    for i, (rows, in_f, out_f, tile) in enumerate(g["gemm_shapes"].tolist()):
        print(f"case gemm{i} rows={rows} in_f={in_f} out_f={out_f} tile={tile}", flush=True)
        x = torch.from_numpy(g[f"gemm{i}_x"]).to(DEV)
        w = torch.from_numpy(g[f"gemm{i}_w"]).to(DEV)
        s = torch.from_numpy(g[f"gemm{i}_s"]).to(DEV)
        y = be().fp8_forward(x, w, s, in_f, out_f, tile)
        ref = torch.from_numpy(g[f"gemm{i}_y"])
        assert y.dtype == torch.float32 and tuple(y.shape) == (rows, out_f)
        # test_linear_fp8.py:170-183 bar: rel < 1e-5 (fp32 x goes through the hi+lo split)
        assert rel_max(y, ref) < 1e-5, (i, rel_max(y, ref))


@pytest.mark.parametrize("rows,in_f,out_f,tile", [(128, 64, 9, 64), (5, 100, 70, 64), (33, 65, 65, 64),
                                                  (64, 512, 256, 64), (300, 256, 200, 32),
                                                  (77, 384, 130, 128), (1, 1024, 64, 64)])
def test_fp8_linear_bf16_inputs_vs_oracle(rows, in_f, out_f, tile):
    print(f"case rows={rows} in_f={in_f} out_f={out_f} tile={tile}", flush=True)
    gen = torch.Generator().manual_seed(rows * 7 + in_f)
    x = torch.randn(rows, in_f, generator=gen).to(torch.bfloat16)
    w, s = oracle.quantize_tiles(torch.randn(out_f, in_f, generator=gen) * 0.02, tile)
    ref = oracle.fp8_forward(x.float(), w, s, in_f, out_f, tile)
    y = be().fp8_forward(x.to(DEV), w.to(DEV), s.to(DEV), in_f, out_f, tile)
    assert rel_max(y, ref) < 2e-6, rel_max(y, ref)


@pytest.mark.parametrize("rows,in_f,out_f,raw_codes", [
    (4096, 512, 1280, False),   # C2 gate: 64x128 tiles
    (4096, 1280, 512, False),   # C2 down: 32x128 tiles
    (300, 256, 384, False),     # ragged last row tile
    (16384, 1024, 2560, False), # 128x256 tiles
    (512, 256, 256, True),      # every code, 0x7F/0xFF decoded on the fly
])
def test_fp8_linear_bf16_dma_tiles(rows, in_f, out_f, raw_codes):
    """bf16 x with 64-wide tiles and out_f a multiple of 128 runs the LDS-DMA
    kernel with fp32 output, its tile sized to the grid.  A sample of rows
    (first, middle, last) against the oracle at the bf16-input bar."""
    print(f"case fp8_linear dma rows={rows} in_f={in_f} out_f={out_f} raw={raw_codes}", flush=True)
    gen = torch.Generator().manual_seed(rows + in_f * 3 + out_f)
    x = torch.randn(rows, in_f, generator=gen).to(torch.bfloat16)
    if raw_codes:
        w = torch.randint(0, 256, (out_f, in_f), generator=gen, dtype=torch.int64).to(torch.uint8)
        s = torch.rand(out_f, in_f // 64, generator=gen) * 0.01 + 1e-3
    else:
        w, s = oracle.quantize_tiles(torch.randn(out_f, in_f, generator=gen) * 0.02, 64)
    y = be().fp8_forward(x.to(DEV), w.to(DEV), s.to(DEV), in_f, out_f, 64).cpu()
    idx = torch.cat([torch.arange(0, min(rows, 96)), torch.arange(rows // 2, rows // 2 + 33),
                     torch.arange(max(0, rows - 65), rows)]).unique()
    ref = oracle.fp8_forward(x[idx].float(), w, s, in_f, out_f, 64)
    assert torch.isfinite(y).all()
    assert rel_max(y[idx], ref) < 2e-6, rel_max(y[idx], ref)


@pytest.mark.parametrize("rows,in_f,out_f,tile", [
    (4096, 512, 1280, 64),      # C2 gate: two bf16 planes through the 64x128 DMA tiles
    (4096, 1280, 512, 64),      # C2 down: 32x128 tiles
    (300, 256, 384, 64),        # ragged last row tile
    (2048, 1024, 2560, 64),     # 128x256 tiles
    (512, 64, 256, 64),         # in-LDS split (<= 1024 rows), one 64-wide K block
    (1000, 1024, 2560, 64),     # in-LDS split, 64x128 tiles
    (1024, 64, 16384, 64),      # in-LDS split, 128x256 tiles
    (700, 256, 384, 64),        # in-LDS split, 32x128 tiles
    (64, 512, 256, 64),         # rows <= 64: the register-staged split kernel
    (512, 256, 200, 64),        # out_f not a multiple of 128: register-staged
    (300, 384, 256, 128),       # tile 128: register-staged
])
def test_fp8_linear_fp32_two_planes(rows, in_f, out_f, tile):
    """fp32 x (what FP8Linear passes) through fp8_forward: split into bf16 hi and
    lo planes (in a workspace pass above 1024 rows, in LDS inside the GEMM
    below) for the LDS-DMA GEMM, or the register-staged kernel where the shape
    does not fit it.  Rows sampled against the oracle at the fp32-input bar
    (test_linear_fp8.py:170-183)."""
    print(f"case fp8_linear fp32 rows={rows} in_f={in_f} out_f={out_f} tile={tile}", flush=True)
    gen = torch.Generator().manual_seed(rows * 5 + in_f + out_f * 7 + tile)
    x = torch.randn(rows, in_f, generator=gen)
    x[0, :7] = torch.tensor([0.0, -0.0, 1e-30, -3e4, 2.0 ** -133, 1.0 + 2.0 ** -20, 65504.0])
    w, s = oracle.quantize_tiles(torch.randn(out_f, in_f, generator=gen) * 0.02, tile)
    y = be().fp8_forward(x.to(DEV), w.to(DEV), s.to(DEV), in_f, out_f, tile).cpu()
    idx = torch.cat([torch.arange(0, min(rows, 96)), torch.arange(rows // 2, min(rows, rows // 2 + 33)),
                     torch.arange(max(0, rows - 65), rows)]).unique()
    ref = oracle.fp8_forward(x[idx], w, s, in_f, out_f, tile)
    assert torch.isfinite(y).all()
    assert rel_max(y[idx], ref) < 1e-5, rel_max(y[idx], ref)


def test_fp8_linear_ws_abi_fallbacks():
    """smaul_fp8_linear_ws through the C-ABI: the two-plane path with a large
    enough workspace and smaul_fp8_linear itself (the in-LDS split) without
    one or with one too small, both within the fp32-input bar of the oracle;
    bf16 x and short fp32 calls need no workspace; the size query."""
    from smaulnative_amd import _lib
    lib = _lib.load()
    rows, in_f, out_f = 2048, 512, 384
    assert lib.smaul_fp8_linear_workspace_size(rows, in_f, _lib.DTYPE_F32) == rows * in_f * 4
    assert lib.smaul_fp8_linear_workspace_size(1024, in_f, _lib.DTYPE_F32) == 0  # in-LDS split instead
    assert lib.smaul_fp8_linear_workspace_size(rows, in_f, _lib.DTYPE_BF16) == 0
    assert lib.smaul_fp8_linear_workspace_size(-1, in_f, _lib.DTYPE_F32) == -1
    gen = torch.Generator().manual_seed(77)
    x = torch.randn(rows, in_f, generator=gen)
    w, s = oracle.quantize_tiles(torch.randn(out_f, in_f, generator=gen) * 0.02, 64)
    ref = oracle.fp8_forward(x[:80], w, s, in_f, out_f, 64)
    xd, wd, sd = x.to(DEV), w.to(DEV), s.to(DEV)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for nbytes in (rows * in_f * 4, rows * in_f * 4 - 16, 0):
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=DEV)
        y = torch.full((rows, out_f), float("nan"), device=DEV)
        rc = lib.smaul_fp8_linear_ws(xd.data_ptr(), _lib.DTYPE_F32, wd.data_ptr(), sd.data_ptr(), y.data_ptr(),
                                     _lib.DTYPE_F32, rows, in_f, out_f, 64, 0,
                                     ws.data_ptr() if nbytes else None, nbytes, stream)
        assert rc == _lib.SMAUL_OK, _lib.last_error()
        torch.cuda.synchronize()
        assert torch.isfinite(y).all()
        assert rel_max(y[:80].cpu(), ref) < 1e-5
        outs.append(y.cpu())
    # the two fallbacks are the same kernel
    assert torch.equal(outs[1], outs[2])
    assert rel_max(outs[0], outs[2]) < 1e-5
    # a bad argument is reported as by smaul_fp8_linear
    rc = lib.smaul_fp8_linear_ws(xd.data_ptr(), _lib.DTYPE_F32, wd.data_ptr(), sd.data_ptr(), None,
                                 _lib.DTYPE_F32, rows, in_f, out_f, 64, 0, None, 0, stream)
    assert rc == _lib.SMAUL_ERR_INVALID


def test_fp8_linear_special_codes():
    # every one of the 256 codes, including 0x7F/0xFF (+-448, NaN in OCP),
    # 0x80 (-0) and the subnormals, against the reference codebook
    in_f, out_f, rows = 256, 64, 32
    codes = torch.arange(256, dtype=torch.int64).repeat(out_f, 1)
    codes = torch.stack([torch.roll(codes[i], i) for i in range(out_f)]).to(torch.uint8)
    gen = torch.Generator().manual_seed(5)
    s = torch.rand(out_f, in_f // 64, generator=gen) * 0.01 + 1e-3
    x = torch.randn(rows, in_f, generator=gen).to(torch.bfloat16)
    ref = oracle.fp8_forward(x.float(), codes, s, in_f, out_f, 64)
    y = be().fp8_forward(x.to(DEV), codes.to(DEV), s.to(DEV), in_f, out_f, 64)
    assert torch.isfinite(y).all()
    assert rel_max(y, ref) < 2e-6


def test_c2_dense_swiglu_pair_full_size_f32():
    """Config 2 with the fp32 activations it specifies: x and then hdn split
    into bf16 hi / lo planes, gate+up with the SwiGLU epilogue kept in fp32,
    down with fp32 output; every 8th row against the oracle at the fp32 bar."""
    gen = torch.Generator().manual_seed(1237)
    rows, d, h = 4096, 512, 1280
    x = torch.randn(rows, d, generator=gen)
    ex = oracle.make_expert(d, h, gen)
    bufs = tuple(t.to(DEV) for t in (ex.gate_w, ex.gate_s, ex.up_w, ex.up_s, ex.down_w, ex.down_s))
    y = be().swiffn_forward(x.to(DEV), bufs, 64).cpu()
    assert y.dtype == torch.float32 and y.shape == x.shape and torch.isfinite(y).all()
    idx = torch.arange(0, rows, 8)
    ref = oracle.swiffn_forward(x[idx], ex)
    err = rel_l2(y[idx], ref)
    print(f"rel_l2={err:.3e}")
    assert err < 1e-5


def test_swiffn_f32_workspace_without_planes():
    """smaul_swiffn_forward through the C-ABI with fp32 x: a workspace of only
    the hdn part (what the size query returned before the planes were added)
    runs the register-staged kernels; the full size takes the planes.  Both
    within the fp32 bar of the oracle."""
    from smaulnative_amd import _lib
    lib = _lib.load()
    gen = torch.Generator().manual_seed(1238)
    rows, d, h = 300, 256, 640
    x = torch.randn(rows, d, generator=gen)
    ex = oracle.make_expert(d, h, gen)
    ref = oracle.swiffn_forward(x, ex)
    xd = x.to(DEV)
    bufs = [t.to(DEV) for t in (ex.gate_w, ex.gate_s, ex.up_w, ex.up_s, ex.down_w, ex.down_s)]
    full = lib.smaul_swiffn_workspace_size(rows, h, _lib.DTYPE_F32)
    part = ((rows * h * 4 + 255) // 256) * 256
    assert full == 2 * part
    for nbytes in (part, full):
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        out = torch.empty(rows, d, device=DEV)
        rc = lib.smaul_swiffn_forward(xd.data_ptr(), _lib.DTYPE_F32, *[t.data_ptr() for t in bufs], out.data_ptr(),
                                      ws.data_ptr(), nbytes, rows, d, h, 64, 0, None)
        _lib.check(rc, "swiffn_forward")
        torch.cuda.synchronize()
        err = rel_l2(out.cpu(), ref)
        print(f"workspace {nbytes}: rel_l2={err:.3e}")
        assert err < 1e-5
    short = torch.empty(part - 256, dtype=torch.uint8, device=DEV)
    assert lib.smaul_swiffn_forward(xd.data_ptr(), _lib.DTYPE_F32, *[t.data_ptr() for t in bufs], out.data_ptr(),
                                    short.data_ptr(), part - 256, rows, d, h, 64, 0, None) != 0


def test_c2_dense_swiglu_pair_full_size():
    """Config 2: 4096 x 512 -> 2 x 1280 (gate and up in one launch with the
    SwiGLU epilogue), then 1280 -> 512, bf16 x, through the fused entry."""
    gen = torch.Generator().manual_seed(1236)
    rows, d, h = 4096, 512, 1280
    x = torch.randn(rows, d, generator=gen).to(torch.bfloat16)
    ex = oracle.make_expert(d, h, gen)
    bufs = tuple(t.to(DEV) for t in (ex.gate_w, ex.gate_s, ex.up_w, ex.up_s, ex.down_w, ex.down_s))
    y = be().swiffn_forward(x.to(DEV), bufs, 64).cpu()
    assert y.dtype == torch.bfloat16 and y.shape == x.shape
    # the oracle (model.py:289-290 with the reference GEMM) on every 8th row
    idx = torch.arange(0, rows, 8)
    ref = oracle.swiffn_forward(x[idx], ex)
    err = rel_l2(y[idx].float(), ref.float())
    print(f"rel_l2={err:.3e}")
    assert err < 2e-3


@pytest.mark.parametrize("rows,d,h,dtype,tile", [
    (37, 256, 640, torch.bfloat16, 64),     # small row count: 32-row register-staged tiles
    (300, 192, 320, torch.bfloat16, 64),    # d not a multiple of 256: register-staged down
    (300, 256, 640, torch.float32, 64),     # fp32 activations: hi / lo planes through the LDS-DMA kernels
    (1000, 1024, 2560, torch.float32, 64),  # the same with 128-row gate+up tiles
    (64, 256, 640, torch.float32, 64),      # fp32, <= 64 rows: register-staged kernels
    (300, 640, 256, torch.float32, 64),     # fp32, d > h: register-staged kernels
    (300, 192, 320, torch.float32, 64),     # fp32, d not a multiple of 128: register-staged kernels
    (129, 256, 512, torch.bfloat16, 32),
    (200, 256, 384, torch.bfloat16, 128),
    (1, 512, 1280, torch.bfloat16, 64),
])
def test_swiffn_dense_vs_oracle(rows, d, h, dtype, tile):
    print(f"case swiffn rows={rows} d={d} h={h} {dtype} tile={tile}", flush=True)
    gen = torch.Generator().manual_seed(rows * 13 + d + h)
    x = torch.randn(rows, d, generator=gen).to(dtype)
    ex = oracle.make_expert(d, h, gen, tile)
    bufs = tuple(t.to(DEV) for t in (ex.gate_w, ex.gate_s, ex.up_w, ex.up_s, ex.down_w, ex.down_s))
    y = be().swiffn_forward(x.to(DEV), bufs, tile).cpu()
    ref = oracle.swiffn_forward(x, ex, tile)
    assert y.dtype == dtype
    err = rel_l2(y.float(), ref.float())
    print(f"rel_l2={err:.3e}")
    assert err < (2e-3 if dtype == torch.bfloat16 else 1e-5)


def test_swiffn_module_on_device():
    """SwiFFN.forward (model.py:289-290) runs the fused entry on the device."""
    from smaulnative_amd import MoEConfig, SwiFFN
    torch.manual_seed(1)
    ffn = SwiFFN(MoEConfig(d_model=256, ffn_mult=2.5)).eval()
    ex = oracle.ExpertWeights(*[t.clone() for t in ffn.buffers6()])
    x = torch.randn(3, 40, 256).to(torch.bfloat16)
    ref = oracle.swiffn_forward(x, ex)
    with torch.no_grad():
        y = ffn.to(DEV)(x.to(DEV)).cpu()
    assert y.shape == x.shape and y.dtype == torch.bfloat16
    assert rel_l2(y.float(), ref.float()) < 2e-3


# --------------------------------------------------------------------------
# router and dispatch
# --------------------------------------------------------------------------
@pytest.mark.parametrize("T,d,E,k,dtype", [(4096, 1024, 8, 2, torch.bfloat16), (2048, 2048, 16, 2, torch.bfloat16),
                                           (1000, 512, 4, 2, torch.float32), (777, 256, 8, 3, torch.bfloat16),
                                           (64, 1024, 8, 2, torch.bfloat16), (300, 64, 1, 1, torch.float32),
                                           (129, 128, 64, 5, torch.bfloat16)])
def test_router_matches_oracle(T, d, E, k, dtype):
    print(f"case router T={T} d={d} E={E} k={k} {dtype}", flush=True)
    gen = torch.Generator().manual_seed(T + d + E)
    x = torch.randn(T, d, generator=gen).to(dtype)
    gw = torch.randn(E, d, generator=gen) * 0.02
    gb = torch.randn(E, generator=gen) * 0.5
    prob_r, topi_r, topw_r = oracle.route(x, gw, gb, k)
    prob, topi, topw = be().moe_router(x.to(DEV), gw.to(DEV), gb.to(DEV), k)
    torch.cuda.synchronize()
    prob, topi, topw = prob.cpu(), topi.cpu(), topw.cpu()
    assert rel_max(prob, prob_r) < 1e-5
    diff = (topi != topi_r).any(1)
    if diff.any():  # printed so that a near-tie flip is diagnosable; none is accepted
        print(f"routing flips: {int(diff.sum())} of {T}, margins {route_margin(prob_r, topi_r, k)[diff].tolist()}")
    assert torch.equal(topi, topi_r)
    assert rel_max(topw, topw_r) < 1e-5


def test_dispatch_permutation_bit_exact():
    gen = torch.Generator().manual_seed(11)
    T, d, E, k = 5000, 256, 8, 2
    x = torch.randn(T, d, generator=gen).to(torch.bfloat16)
    gw = torch.randn(E, d, generator=gen) * 0.05
    gb = torch.tensor([2.0, 0, 0, 0, 0, -3.0, -3.0, 0])
    b = be()
    prob, topi, topw = b.moe_router(x.to(DEV), gw.to(DEV), gb.to(DEV), k)
    disp = b.moe_dispatch(topi, topw, E)
    torch.cuda.synchronize()
    topi_c, topw_c = topi.cpu(), topw.cpu()
    counts = disp["counts"].cpu().tolist()
    seg = disp["seg_off"].cpu().tolist()
    perm = disp["perm_row"].cpu()
    pw = disp["perm_w"].cpu()
    inv = disp["inv"].cpu().reshape(T, k)
    # brute force from the same topi/topw: for each expert, ascending tokens with w > 0
    for e in range(E):
        w_e = torch.where(topi_c == e, topw_c, torch.zeros_like(topw_c)).sum(-1)
        toks = torch.nonzero(w_e > 0).flatten()
        assert counts[e] == toks.numel()
        assert seg[e + 1] - seg[e] == toks.numel()
        assert torch.equal(perm[seg[e]:seg[e + 1]].long(), toks)
        assert torch.equal(pw[seg[e]:seg[e + 1]], w_e[toks])
    for t in range(0, T, 97):
        for j in range(k):
            pos = int(inv[t, j])
            assert pos >= 0 and int(perm[pos]) == t
    bm = disp["block_m"]
    tiles = disp["tile_off"].cpu().tolist()
    assert tiles == [sum((c + bm - 1) // bm for c in counts[:e]) for e in range(E + 1)]


@pytest.mark.parametrize("T,E,k", [(20000, 8, 2), (20000, 16, 3), (70000, 4, 1)])
def test_dispatch_many_blocks_bit_exact(T, E, k):
    """Past 256 router blocks the dispatch scan runs as its own kernel: the
    permutation, counts and inverse map still follow the brute-force order."""
    print(f"case dispatch T={T} E={E} k={k}", flush=True)
    gen = torch.Generator().manual_seed(T + E)
    topi = torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(T)]).to(torch.int64)
    topw = torch.rand(T, k, generator=gen)
    topw[torch.rand(T, k, generator=gen) < 0.05] = 0.0  # w == 0: not dispatched (model.py:576)
    disp = be().moe_dispatch(topi.to(DEV), topw.to(DEV), E, 128)
    torch.cuda.synchronize()
    counts = disp["counts"].cpu().tolist()
    seg = disp["seg_off"].cpu().tolist()
    perm = disp["perm_row"].cpu()
    pw = disp["perm_w"].cpu()
    inv = disp["inv"].cpu().reshape(T, k)
    for e in range(E):
        w_e = torch.where(topi == e, topw, torch.zeros_like(topw)).sum(-1)
        toks = torch.nonzero(w_e > 0).flatten()
        assert counts[e] == toks.numel() and seg[e + 1] - seg[e] == toks.numel()
        assert torch.equal(perm[seg[e]:seg[e + 1]].long(), toks)
        assert torch.equal(pw[seg[e]:seg[e + 1]], w_e[toks])
    live = topw > 0
    assert bool((inv[~live] == -1).all())
    pos = inv[live].long()
    assert torch.equal(perm[pos].long(), torch.arange(T).unsqueeze(1).expand(T, k)[live])


def test_moe_fp32_many_router_blocks():
    """fp32 activations at E = 16 route 16 tokens per block: T = 4500 gives 282
    blocks, past the fused scan + scatter kernel's 256."""
    print("case moe fp32 T=4500 E=16", flush=True)
    T, d, h, E, k = 4500, 128, 256, 16, 2
    x, gw, gb, experts = make_moe(4500, T, d, h, E, k, dtype=torch.float32)
    ref = oracle.moe_forward(x, gw, gb, experts, k)
    out, prob, topi, counts = gpu_moe(x, gw, gb, experts, k)
    assert torch.equal(topi, ref.topi)
    assert counts.tolist() == ref.counts
    assert rel_l2(out, ref.out) < 1e-5


def test_host_tensors_rejected_before_launch():
    """A bias, norm weight or routing tensor left on the host raises in Python;
    no host pointer reaches a kernel."""
    x, gw, gb, experts = make_moe(3, 64, 128, 256, 4, 2)
    b = be()
    xd, gwd, exd = x.to(DEV), gw.to(DEV), to_dev_experts(experts)
    with pytest.raises(RuntimeError, match="HIP device"):
        b.moe_forward(xd, gwd, gb, exd, 2, 64)
    with pytest.raises(RuntimeError, match="HIP device"):
        b.moe_forward_norm(xd, gwd, gb.to(DEV), exd, 2, 64, torch.ones(128), 1e-6)
    with pytest.raises(RuntimeError, match="HIP device"):
        b.moe_router(xd, gwd, gb, 2)
    with pytest.raises(RuntimeError, match="HIP device"):
        b.moe_stages(xd, gwd, gb, exd, 2, 64)
    prob, topi, topw = b.moe_router(xd, gwd, gb.to(DEV), 2)
    with pytest.raises(RuntimeError, match="HIP device"):
        b.moe_dispatch(topi, topw.cpu(), 4)


# --------------------------------------------------------------------------
# whole MoE layer
# --------------------------------------------------------------------------
def _golden_case(g, tag):
    from _cases import load_moe_case
    return load_moe_case(g, tag)


@pytest.mark.parametrize("tag", ["moe_e4k2_f32", "moe_e4k2_bf16", "moe_e8k3_bf16", "moe_e8k2_bf16",
                                 "moe_tie_uniform", "moe_tie_underflow", "moe_zero_weight"])
def test_moe_golden(tag):
    print(f"case {tag}", flush=True)
    g = np.load(GOLD)
    c = _golden_case(g, tag)
    out, prob, topi, counts = gpu_moe(c["x"], c["gate_w"], None, c["experts"], c["k"], c["tile"])
    assert torch.equal(topi, c["topi"]), (tag, topi.reshape(-1, c["k"])[:4], c["topi"].reshape(-1, c["k"])[:4])
    assert counts.tolist() == c["counts"]
    assert rel_max(prob, c["prob"]) < 1e-5
    assert out.dtype == c["out"].dtype and out.shape == c["out"].shape
    assert rel_l2(out.float(), c["out"].float()) < 2e-3, rel_l2(out.float(), c["out"].float())


@pytest.mark.parametrize("T,d,h,E,k,dtype,tile", [
    (1024, 1024, 2560, 8, 2, torch.bfloat16, 64),      # config-3 shape, fewer tokens
    (600, 256, 640, 8, 3, torch.bfloat16, 64),
    (512, 512, 1280, 4, 2, torch.bfloat16, 64),        # config-1 MoE layer shape
    (333, 256, 640, 8, 2, torch.float32, 64),          # fp32 x: hi / lo planes, 64-row LDS-DMA tiles
    (4096, 1024, 2560, 8, 2, torch.float32, 64),       # fp32 x: planes, 128-row tiles, 128x128 down
    (2048, 512, 1024, 8, 2, torch.float32, 64),        # fp32 x: planes, 128x256 down tiles
    (40, 256, 640, 4, 2, torch.float32, 64),           # fp32 x, decode-sized: planes on 64-row tiles
    (300, 192, 640, 4, 2, torch.float32, 64),          # fp32 x, d not a multiple of 128: register-staged
    (256, 256, 512, 4, 1, torch.bfloat16, 128),
    (200, 128, 320, 2, 2, torch.bfloat16, 32),
    (64, 1024, 2560, 8, 2, torch.bfloat16, 64),        # config-4 decode-sized step
    (17, 64, 160, 1, 1, torch.bfloat16, 64),
    (300, 256, 384, 2, 1, torch.bfloat16, 64),         # 64-row tiles: two experts, top-1
    (1000, 128, 256, 3, 2, torch.bfloat16, 64),        # 64-row tiles: K = 128 (two stages)
])
def test_moe_vs_oracle(T, d, h, E, k, dtype, tile):
    print(f"case moe T={T} d={d} h={h} E={E} k={k} {dtype} tile={tile}", flush=True)
    x, gw, gb, experts = make_moe(T * 3 + d, T, d, h, E, k, dtype, tile=tile)
    ref = oracle.moe_forward(x, gw, gb, experts, k, tile)
    out, prob, topi, counts = gpu_moe(x, gw, gb, experts, k, tile)
    diff = (topi.reshape(-1, k) != ref.topi.reshape(-1, k)).any(1)
    if diff.any():  # printed so that a near-tie flip is diagnosable; none is accepted
        print(f"routing flips: {int(diff.sum())}, margins {route_margin(ref.prob, ref.topi, k)[diff].tolist()}")
    assert torch.equal(topi.reshape(-1, k), ref.topi.reshape(-1, k))
    assert counts.tolist() == ref.counts
    err = rel_l2(out.float(), ref.out.float())
    print(f"rel_l2={err:.3e}")
    assert err < (2e-3 if dtype == torch.bfloat16 else 1e-5)


@pytest.mark.parametrize("T,E,k,skew", [(1, 4, 2, None), (5, 8, 2, None), (33, 8, 3, None), (64, 16, 2, None),
                                         (64, 8, 2, (9.0, [], 0.0)), (48, 4, 1, None)])
def test_moe_decode_regime(T, E, k, skew):
    """T <= 64 runs the decode kernels (weights streamed once per expert)."""
    print(f"case decode T={T} E={E} k={k} skew={skew}", flush=True)
    d, h = 256, 640
    x, gw, gb, experts = make_moe(T * 7 + E, T, d, h, E, k, skew=skew)
    ref = oracle.moe_forward(x, gw, gb, experts, k)
    out, prob, topi, counts = gpu_moe(x, gw, gb, experts, k)
    assert torch.equal(topi.reshape(-1, k), ref.topi.reshape(-1, k))
    assert counts.tolist() == ref.counts
    if skew is not None:
        assert max(ref.counts) == T  # every token picked expert 0: 4 row tiles of 16
    assert rel_l2(out.float(), ref.out.float()) < 2e-3


@pytest.mark.parametrize("T,skew", [(64, (9.0, [], 0.0)), (40, (9.0, [3, 4, 5, 6, 7], 9.0)), (7, None)])
def test_moe_decode_c4_shape(T, skew):
    """Config-4 widths in the decode regime: one expert holding every token
    (four 16-row tiles), experts left idle (no segment, no unit), and a tiny
    step."""
    print(f"case decode c4 T={T} skew={skew}", flush=True)
    d, h, E, k = 1024, 2560, 8, 2
    x, gw, gb, experts = make_moe(640 + T, T, d, h, E, k, skew=skew)
    ref = oracle.moe_forward(x, gw, gb, experts, k)
    out, prob, topi, counts = gpu_moe(x, gw, gb, experts, k)
    assert torch.equal(topi.reshape(-1, k), ref.topi.reshape(-1, k))
    assert counts.tolist() == ref.counts
    if skew is not None:
        assert max(ref.counts) == T
    err = rel_l2(out.float(), ref.out.float())
    print(f"counts {ref.counts} rel_l2={err:.3e}")
    assert err < 2e-3


def test_moe_skewed_segments():
    """Config-5 style skew (one expert ~40 %, three < 1 %) at a reduced size."""
    x, gw, gb, experts = make_moe(55, 2048, 256, 640, 16, 2, skew=(2.2, [13, 14, 15], 4.0))
    ref = oracle.moe_forward(x, gw, gb, experts, 2, 64)
    out, prob, topi, counts = gpu_moe(x, gw, gb, experts, 2, 64)
    print("counts", counts.tolist())
    assert counts.tolist() == ref.counts
    assert max(ref.counts) > 0.3 * 2 * 2048
    assert rel_l2(out.float(), ref.out.float()) < 2e-3


@pytest.mark.parametrize("T,d,h", [(900, 512, 1280), (64, 1024, 2560), (5, 256, 640), (17, 1024, 2560),
                                   (20, 1024, 1024)])
def test_staged_call_equals_fused_call(T, d, h):
    """The five stage entries and the single-call layer give identical bits.
    At decode sizes the single call routes with one router block per 16 tokens
    (the stage entry uses 64-token blocks), its gate/up kernel dispatches for
    itself and (d = 1024: 8-wave down instances, 5 or 2 K blocks per wave) the
    combine runs in the down kernel's tail, so this also checks that none of
    them changes a bit; T = 17 leaves the last combining workgroup one token."""
    print(f"case staged T={T} d={d} h={h}", flush=True)
    x, gw, gb, experts = make_moe(91, T, d, h, 8, 2)
    b = be()
    exd = to_dev_experts(experts)
    out, prob, topi, counts = b.moe_forward(x.to(DEV), gw.to(DEV), gb.to(DEV), exd, 2, 64)
    out2, prob2, topi2, topw2, disp = b.moe_stages(x.to(DEV), gw.to(DEV), gb.to(DEV), exd, 2, 64)
    torch.cuda.synchronize()
    assert torch.equal(out, out2) and torch.equal(prob, prob2) and torch.equal(topi, topi2)
    assert torch.equal(counts, disp["counts"])


@pytest.mark.parametrize("T,d,h,E,k", [(900, 512, 1280, 8, 2), (3000, 1024, 2560, 8, 2), (300, 256, 384, 2, 1)])
def test_stage_entries_block_m_64(T, d, h, E, k):
    """The stage entries on 64-row tiles (block_m 64, which moe_forward takes
    for small layers) give the bits of 128-row tiles, whatever moe_forward
    picks for the shape (T = 3000 at d = 1024: above its 64-row threshold)."""
    print(f"case stages block_m 64 T={T} d={d} h={h} E={E} k={k}", flush=True)
    x, gw, gb, experts = make_moe(5 + T, T, d, h, E, k)
    b = be()
    exd = to_dev_experts(experts)
    args = (x.to(DEV), gw.to(DEV), gb.to(DEV), exd, k, 64)
    o64 = b.moe_stages(*args, block_m=64)[0]
    o128 = b.moe_stages(*args, block_m=128)[0]
    of = b.moe_forward(*args)[0]
    torch.cuda.synchronize()
    assert torch.equal(o64, o128) and torch.equal(o64, of)


def test_moe_64_row_tiles_empty_experts():
    """64-row tiles with five of eight experts never chosen (empty segments)
    and one expert holding most rows."""
    print("case 64-row tiles, empty experts", flush=True)
    T, d, h, E, k = 700, 256, 384, 8, 2
    x, gw, gb, experts = make_moe(7, T, d, h, E, k, skew=(9.0, [3, 4, 5, 6, 7], 9.0))
    ref = oracle.moe_forward(x, gw, gb, experts, k)
    out, prob, topi, counts = gpu_moe(x, gw, gb, experts, k)
    assert torch.equal(topi.reshape(-1, k), ref.topi.reshape(-1, k))
    assert counts.tolist() == ref.counts
    assert ref.counts[3:] == [0] * 5 and max(ref.counts) == T
    assert rel_l2(out.float(), ref.out.float()) < 2e-3


def test_moe_decode_unsplit_k():
    """K/64 = 18 blocks fits no streaming split (2, 4 or 5 blocks per wave over
    at most 8 waves): both projections run the split-K decode kernel."""
    print("case decode d=h=1152", flush=True)
    T, d, h, E, k = 40, 1152, 1152, 4, 2
    x, gw, gb, experts = make_moe(1152, T, d, h, E, k)
    ref = oracle.moe_forward(x, gw, gb, experts, k)
    out, prob, topi, counts = gpu_moe(x, gw, gb, experts, k)
    assert torch.equal(topi.reshape(-1, k), ref.topi.reshape(-1, k))
    assert counts.tolist() == ref.counts
    assert rel_l2(out.float(), ref.out.float()) < 2e-3


def abi_moe(x, gw, gb, experts, k, tile, flags, code_tensors=None):
    """smaul_moe_forward through the C-ABI on the caller's own code buffers."""
    from smaulnative_amd import _lib
    lib = _lib.load()
    T, d = x.shape
    E = len(experts)
    ex = code_tensors or to_dev_experts(experts)
    h = ex[0][0].shape[0]
    table = torch.tensor([[int(ex[e][j].data_ptr()) for e in range(E)] for j in range(6)],
                         dtype=torch.int64, device=DEV)
    xd, gwd = x.to(DEV).contiguous(), gw.to(DEV).float().contiguous()
    gbd = None if gb is None else gb.to(DEV).float().contiguous()
    out = torch.empty_like(xd)
    prob = torch.empty(T, E, device=DEV)
    topi = torch.empty(T, k, dtype=torch.int64, device=DEV)
    topw = torch.empty(T, k, device=DEV)
    counts = torch.empty(E, dtype=torch.int32, device=DEV)
    act = 1 if x.dtype == torch.bfloat16 else 0
    ws_bytes = lib.smaul_moe_workspace_size(T, d, h, E, k, act)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    tp, row = table.data_ptr(), E * 8
    rc = lib.smaul_moe_forward(xd.data_ptr(), act, gwd.data_ptr(), None if gbd is None else gbd.data_ptr(),
                               tp, tp + row, tp + 2 * row, tp + 3 * row, tp + 4 * row, tp + 5 * row,
                               out.data_ptr(), prob.data_ptr(), topi.data_ptr(), topw.data_ptr(),
                               counts.data_ptr(), ws.data_ptr(), ws_bytes, T, d, h, E, k, tile, flags,
                               torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "moe_forward")
    torch.cuda.synchronize()
    return out.cpu(), topi.cpu(), counts.cpu()


@pytest.mark.parametrize("T,flags,block_m", [(1024, 0, 128), (1024, 2, 128), (64, 0, 16)])
def test_moe_raw_codes_any_flags(T, flags, block_m):
    """Raw stored codes (0x7F/0xFF included, no canonical copy).  At 128-row
    tiles without SMAUL_FLAG_ALIGNED_CODES the register-staged kernels run;
    with it the LDS-DMA kernels decode 0x7F/0xFF themselves; T = 64 runs the
    decode kernels on the raw codes."""
    from smaulnative_amd import _lib
    print(f"case raw codes T={T} flags={flags}", flush=True)
    d, h, E, k = 1024, 2560, 8, 2
    x, gw, gb, experts = make_moe(4242 + T, T, d, h, E, k)
    assert _lib.load().smaul_moe_block_m(T, d, h, E, k, 64, 1) == block_m
    gen = torch.Generator().manual_seed(5)
    for ex in experts:   # plant 0x7F (= 448, like 0x7E) where the quantizer chose 0x7E
        for w in (ex.gate_w, ex.up_w, ex.down_w):
            m = (w == 0x7E) & (torch.rand(w.shape, generator=gen) < 0.5)
            w[m] = 0x7F
    n7f = sum(int((w == 0x7F).sum()) for ex in experts for w in (ex.gate_w, ex.up_w, ex.down_w))
    nff = sum(int((w == 0xFF).sum()) for ex in experts for w in (ex.gate_w, ex.up_w, ex.down_w))
    assert n7f > 0 and nff > 0
    ref = oracle.moe_forward(x, gw, gb, experts, k, 64)
    out, topi, counts = abi_moe(x, gw, gb, experts, k, 64, flags)
    assert torch.equal(topi, ref.topi.reshape(-1, k))
    assert counts.tolist() == ref.counts
    err = rel_l2(out.float(), ref.out.float())
    print(f"rel_l2={err:.3e} (0x7F codes {n7f}, 0xFF codes {nff})")
    assert err < 2e-3


@pytest.mark.parametrize("T,d,h,layout", [(700, 512, 1280, "raw"), (700, 512, 1280, "raw-aligned"),
                                           (8192, 256, 1024, "raw-aligned"), (700, 512, 1280, "tiled"),
                                           (8192, 256, 1024, "tiled")])
def test_moe_fp32_x_abi_layouts(T, d, h, layout):
    """fp32 x through the C-ABI on the caller's buffers: raw stored codes
    (0x7F/0xFF included) without SMAUL_FLAG_ALIGNED_CODES run the
    register-staged kernels; with it, and with tiled canonical copies, the
    LDS-DMA kernels over bf16 hi / lo planes (64-row tiles at T = 700, 128-row
    at T = 8192).  All within the fp32 bar of the oracle."""
    from smaulnative_amd import _lib
    print(f"case moe fp32 abi T={T} d={d} h={h} {layout}", flush=True)
    E, k = 8, 2
    x, gw, gb, experts = make_moe(777 + T, T, d, h, E, k, dtype=torch.float32)
    gen = torch.Generator().manual_seed(6)
    for ex in experts:   # 0x7F (= 448, like 0x7E) where the quantizer chose 0x7E
        for w in (ex.gate_w, ex.up_w, ex.down_w):
            w[(w == 0x7E) & (torch.rand(w.shape, generator=gen) < 0.5)] = 0x7F
    ref = oracle.moe_forward(x, gw, gb, experts, k, 64)
    if layout == "tiled":
        flags = _lib.FLAG_TILED_LAYOUT | _lib.FLAG_CANONICAL_CODES | _lib.FLAG_ALIGNED_CODES
        out, topi, counts = abi_moe(x, gw, gb, experts, k, 64, flags, tiled_copies(to_dev_experts(experts)))
    else:
        flags = _lib.FLAG_ALIGNED_CODES if layout == "raw-aligned" else 0
        out, topi, counts = abi_moe(x, gw, gb, experts, k, 64, flags)
    assert torch.equal(topi, ref.topi.reshape(-1, k))
    assert counts.tolist() == ref.counts
    err = rel_l2(out, ref.out)
    print(f"rel_l2={err:.3e}")
    assert err < 1e-5


def tiled_copies(ex_dev):
    """The experts' buffers rewritten by smaul_fp8_tile_layout (canonical codes)."""
    from smaulnative_amd import _lib
    lib = _lib.load()
    out = []
    for bufs in ex_dev:
        t = []
        for j in range(0, 6, 2):
            codes, sc = bufs[j], bufs[j + 1].float().contiguous()
            N, K = codes.shape
            c2 = torch.empty_like(codes)
            s2 = torch.empty_like(sc)
            rc = lib.smaul_fp8_tile_layout(codes.data_ptr(), sc.data_ptr(), c2.data_ptr(), s2.data_ptr(), N, K,
                                           torch.cuda.current_stream().cuda_stream)
            _lib.check(rc, "fp8_tile_layout")
            t += [c2, s2]
        out.append(tuple(t))
    return out


def test_tile_layout_entry():
    """smaul_fp8_tile_layout: codes [K/64][N][64] canonical, scales [K/64][N]."""
    gen = torch.Generator().manual_seed(31)
    N, K = 96, 320
    codes = torch.randint(0, 256, (N, K), generator=gen, dtype=torch.uint8)
    codes[0, :4] = torch.tensor([0x7F, 0xFF, 0x7E, 0xFE], dtype=torch.uint8)
    sc = torch.rand(N, K // 64, generator=gen)
    (c2, s2, _, _, _, _), = tiled_copies([(codes.to(DEV), sc.to(DEV)) * 3])
    canon = torch.where((codes & 0x7F) == 0x7F, codes - 1, codes)
    assert torch.equal(c2.cpu().reshape(-1), canon.reshape(N, K // 64, 64).permute(1, 0, 2).reshape(-1))
    assert torch.equal(s2.cpu().reshape(-1), sc.t().reshape(-1))
    # input and output in adjacent halves of one allocation: accepted (only
    # overlapping ranges are rejected), same result
    from smaulnative_amd import _lib
    lib = _lib.load()
    nc, ns = N * K, N * (K // 64)
    cb = torch.zeros(2 * nc, dtype=torch.uint8, device=DEV)
    sb = torch.zeros(2 * ns, dtype=torch.float32, device=DEV)
    cb[:nc] = codes.reshape(-1).to(DEV)
    sb[:ns] = sc.reshape(-1).to(DEV)
    rc = lib.smaul_fp8_tile_layout(cb.data_ptr(), sb.data_ptr(), cb.data_ptr() + nc, sb.data_ptr() + ns * 4, N, K,
                                   torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "fp8_tile_layout")
    torch.cuda.synchronize()
    assert torch.equal(cb[nc:].cpu(), c2.cpu().reshape(-1)) and torch.equal(sb[ns:].cpu(), s2.cpu().reshape(-1))
    assert torch.equal(cb[:nc].cpu(), codes.reshape(-1))  # the input is left as it was


@pytest.mark.parametrize("T,d,h,E,k,dtype", [
    (900, 512, 1280, 8, 2, torch.bfloat16),    # prefill: the LDS-DMA grouped GEMMs
    (300, 256, 640, 8, 2, torch.float32),      # fp32 activations: the register-staged GEMMs
    (200, 256, 640, 16, 2, torch.bfloat16),    # short segments: 32-row register-staged tiles
    (64, 1024, 2560, 8, 2, torch.bfloat16),    # decode: streaming kernels, combine in the down tail
    (20, 1024, 1024, 8, 2, torch.bfloat16),    # decode, the 2-block down instance
    (40, 256, 640, 8, 2, torch.bfloat16),      # decode, 2-wave streaming instances
    (40, 1152, 1152, 4, 2, torch.bfloat16),    # decode, the split-K fallback kernel (18 K blocks)
])
def test_tiled_layout_equals_reference_layout(T, d, h, E, k, dtype):
    """The same layer through the C-ABI on FP8Linear's layout (raw codes) and on
    the tiled copies (SMAUL_FLAG_TILED_LAYOUT): identical bits."""
    from smaulnative_amd import _lib
    lib = _lib.load()
    act = 1 if dtype == torch.bfloat16 else 0
    bm = lib.smaul_moe_block_m(T, d, h, E, k, 64, act)
    print(f"case tiled layout T={T} d={d} h={h} E={E} k={k} {dtype} block_m={bm}", flush=True)
    x, gw, gb, experts = make_moe(5150 + T + d, T, d, h, E, k, dtype)
    ex = to_dev_experts(experts)
    ref = abi_moe(x, gw, gb, experts, k, 64, _lib.FLAG_ALIGNED_CODES, ex)
    flags = _lib.FLAG_CANONICAL_CODES | _lib.FLAG_ALIGNED_CODES | _lib.FLAG_TILED_LAYOUT
    got = abi_moe(x, gw, gb, experts, k, 64, flags, tiled_copies(ex))
    for a, b in zip(ref, got):
        assert torch.equal(a, b)


@pytest.mark.parametrize("rows,d,h", [(300, 256, 640), (4096, 512, 1280), (37, 256, 640)])
def test_swiffn_tiled_layout_equals_reference_layout(rows, d, h):
    from smaulnative_amd import _lib
    lib = _lib.load()
    print(f"case swiffn tiled layout rows={rows} d={d} h={h}", flush=True)
    gen = torch.Generator().manual_seed(rows + d)
    x = torch.randn(rows, d, generator=gen).to(torch.bfloat16).to(DEV)
    ex = oracle.make_expert(d, h, gen)
    bufs = [t.to(DEV) for t in (ex.gate_w, ex.gate_s, ex.up_w, ex.up_s, ex.down_w, ex.down_s)]
    tiled = tiled_copies([bufs])[0]
    outs = []
    for b, flags in ((bufs, _lib.FLAG_ALIGNED_CODES),
                     (tiled, _lib.FLAG_CANONICAL_CODES | _lib.FLAG_ALIGNED_CODES | _lib.FLAG_TILED_LAYOUT)):
        out = torch.empty_like(x)
        ws_bytes = lib.smaul_swiffn_workspace_size(rows, h, 1)
        ws = torch.empty(max(1, ws_bytes), dtype=torch.uint8, device=DEV)
        rc = lib.smaul_swiffn_forward(x.data_ptr(), 1, *[t.data_ptr() for t in b], out.data_ptr(), ws.data_ptr(),
                                      ws_bytes, rows, d, h, 64, flags, torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "swiffn_forward")
        outs.append(out.cpu())
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("d,h,tile,tiled", [(256, 640, 64, True), (256, 640, 32, False), (208, 640, 64, False)])
def test_expert_cache_layout_choice(d, h, tile, tiled):
    """RocmBackend's expert cache writes the tiled layout (and says so in its
    flags) only for tile 64 with d, h multiples of 64; the tiled copies hold
    what smaul_fp8_tile_layout writes, and the layer matches the oracle either
    way."""
    from smaulnative_amd import _lib
    print(f"case expert cache d={d} h={h} tile={tile}", flush=True)
    x, gw, gb, experts = make_moe(6060 + d + tile, 300, d, h, 4, 2, tile=tile)
    ex = to_dev_experts(experts)
    ent = be()._expert_entry(ex, ex[0][0].device, d, h, tile)
    assert bool(ent["flags"] & _lib.FLAG_TILED_LAYOUT) == tiled
    assert ent["flags"] & _lib.FLAG_CANONICAL_CODES and ent["flags"] & _lib.FLAG_ALIGNED_CODES
    if tiled:
        want = tiled_copies(ex)
        for e in range(len(ex)):
            for j in range(6):
                got = ent["copies"][e * 6 + j]
                assert got is not None and torch.equal(got.reshape(-1), want[e][j].reshape(-1))
    ref = oracle.moe_forward(x, gw, gb, experts, 2, tile)
    out, prob, topi, counts = gpu_moe(x, gw, gb, experts, 2, tile)
    assert torch.equal(topi.reshape(-1, 2), ref.topi.reshape(-1, 2))
    assert rel_l2(out.float(), ref.out.float()) < 2e-3


def test_expert_cache_entries_released():
    """An expert-cache entry lives only while the cache holds it: a buffer
    whose storage is swapped (``sc.data = ...``, a new address for the same
    tensor) drops the entry made for its old storage, and freeing a buffer
    drops its entry; neither keeps the copies alive through the finalizers."""
    import gc
    import weakref
    print("case expert cache entries released", flush=True)
    d, h = 256, 640
    _, _, _, experts = make_moe(5151, 8, d, h, 2, 1)
    ex = [list(e) for e in to_dev_experts(experts)]
    b = be()
    old = weakref.ref(b._expert_entry(ex, ex[0][0].device, d, h, 64))
    ex[0][1].data = ex[0][1].data.clone()  # new storage, same tensor object
    new = weakref.ref(b._expert_entry(ex, ex[0][0].device, d, h, 64))
    gc.collect()
    assert old() is None and new() is not None
    del ex[1]
    ex[0] = None
    gc.collect()
    assert new() is None


def test_tiled_layout_rejected_where_unsupported():
    """The tiled flag needs tile 64 and widths that are multiples of 64, and
    smaul_fp8_linear never takes it."""
    from smaulnative_amd import _lib
    lib = _lib.load()
    flags = _lib.FLAG_ALIGNED_CODES | _lib.FLAG_TILED_LAYOUT
    x = torch.zeros(4, 64, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(64, 64, dtype=torch.uint8, device=DEV)
    s = torch.ones(64, 2, device=DEV)
    y = torch.empty(4, 64, device=DEV)
    rc = lib.smaul_fp8_linear(x.data_ptr(), 1, w.data_ptr(), s.data_ptr(), y.data_ptr(), 0, 4, 64, 64, 32, flags,
                              torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.SMAUL_ERR_INVALID
    ws = torch.empty(1 << 16, dtype=torch.uint8, device=DEV)
    rc = lib.smaul_swiffn_forward(x.data_ptr(), 1, w.data_ptr(), s.data_ptr(), w.data_ptr(), s.data_ptr(),
                                  w.data_ptr(), s.data_ptr(), y.data_ptr(), ws.data_ptr(), 1 << 16, 4, 64, 64, 32,
                                  flags, torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.SMAUL_ERR_INVALID


@pytest.mark.parametrize("T,d,k", [(37, 24, 3), (100, 1040, 2), (5, 2048, 4),
                                   (29, 64, 8), (50, 128, 7)])  # every slot order of the sorting network
def test_combine_entry_direct(T, d, k):
    """smaul_moe_combine on its own (16 columns per thread, or 8 when d % 16
    != 0): ascending expert order, fp32 sum from +0 of rounded products,
    slots with inv < 0 skipped."""
    from smaulnative_amd import _lib
    print(f"case combine T={T} d={d} k={k}", flush=True)
    lib = _lib.load()
    gen = torch.Generator().manual_seed(T * d + k)
    E = 8
    topi = torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(T)]).to(torch.int64)
    topw = torch.rand(T, k, generator=gen)
    R = T * k
    perm = torch.randperm(R, generator=gen).to(torch.int32)
    inv = perm.reshape(T, k).clone()
    inv[torch.rand(T, k, generator=gen) < 0.15] = -1
    yperm = torch.randn(R, d, generator=gen).to(torch.bfloat16)
    ref = torch.zeros(T, d)
    for t in range(T):
        acc = torch.zeros(d)
        for j in sorted(range(k), key=lambda j: int(topi[t, j])):
            if inv[t, j] >= 0:
                acc = acc + yperm[int(inv[t, j])].float() * topw[t, j]
        ref[t] = acc
    out = torch.empty(T, d, dtype=torch.bfloat16, device=DEV)
    yd, ti, tw, iv = yperm.to(DEV), topi.to(DEV), topw.to(DEV), inv.to(DEV)
    rc = lib.smaul_moe_combine(yd.data_ptr(), 1, ti.data_ptr(), tw.data_ptr(), iv.data_ptr(), out.data_ptr(),
                               T, d, k, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "moe_combine")
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), ref.to(torch.bfloat16))


def test_moe_deterministic_and_empty():
    x, gw, gb, experts = make_moe(77, 700, 256, 640, 8, 2)
    a = gpu_moe(x, gw, gb, experts, 2)
    b = gpu_moe(x, gw, gb, experts, 2)
    for u, v in zip(a, b):
        assert torch.equal(u, v)
    out, prob, topi, counts = gpu_moe(x[:0], gw, gb, experts, 2)
    assert out.shape == (0, 256) and counts.tolist() == [0] * 8


def test_moe_full_config3():
    """Config 3 at full size: the routing of all 16384 tokens and the per-expert
    counts bit-exact against the oracle router (model.py:558-570, 577); the
    output of a token sample against the oracle's expert loop (tokens are
    independent)."""
    T, d, h, E, k = 16384, 1024, 2560, 8, 2
    x, gw, gb, experts = make_moe(1236, T, d, h, E, k)
    out, prob, topi, counts = gpu_moe(x, gw, gb, experts, k)
    prob_r, topi_r, topw_r = oracle.route(x, gw, gb, k)
    assert torch.equal(topi, topi_r)
    assert counts.tolist() == [int(((topi_r == e) & (topw_r > 0)).any(-1).sum()) for e in range(E)]
    assert rel_max(prob, prob_r) < 1e-5
    idx = torch.arange(0, T, 61)
    ref = oracle.moe_forward(x[idx], gw, gb, experts, k)
    assert torch.equal(topi[idx], ref.topi)
    assert rel_l2(out[idx].float(), ref.out.float()) < 2e-3


def test_swiffn_moe_module_on_device():
    from smaulnative_amd import MoEConfig, SwiFFN_MoE
    torch.manual_seed(0)
    cfg = MoEConfig(d_model=256, ffn_mult=2.5, num_experts=4, num_experts_per_tok=2)
    moe = SwiFFN_MoE(cfg).eval()
    x = torch.randn(2, 50, 256).to(torch.bfloat16)
    experts = []
    for ex in moe.experts:
        experts.append(oracle.ExpertWeights(*[t.clone() for t in ex.buffers6()]))
    gw = moe.gate.weight.detach().clone()
    ref = oracle.moe_forward(x, gw, None, experts, 2, 64)
    moe = moe.to(DEV)
    with torch.no_grad():
        y = moe(x.to(DEV))
    assert y.dtype == torch.bfloat16 and y.shape == x.shape
    assert torch.equal(moe.last_topi.cpu(), ref.topi)
    assert moe.expert_token_counts == ref.counts
    assert moe.last_executed == ref.executed
    st = moe.routing_stats()
    assert sum(st["token_counts"]) == 2 * 50 * 2
    assert rel_l2(y.cpu().float(), ref.out.float()) < 2e-3


@pytest.mark.parametrize("T,d,dtype,weighted", [
    (64, 1024, torch.bfloat16, False),   # the C4 inter-layer norm
    (37, 1000, torch.bfloat16, True),    # 16-byte vectors, ragged last vector per lane
    (5, 1001, torch.bfloat16, False),    # d not a multiple of 8: element path
    (3, 4100, torch.float32, True),      # past the vectors kept in registers
    (2, 8192, torch.bfloat16, True),
    (0, 512, torch.bfloat16, False),
])
def test_rms_norm(T, d, dtype, weighted):
    """RMSNorm.forward (model.py:131-139): (x * rsqrt(mean(x^2) + eps)) * weight
    in fp32, cast to x's dtype.  The row sum is reduced in another order than
    torch's, so bf16 outputs may differ by one ulp on rounding ties and fp32
    outputs by a few ulp."""
    print(f"case rms_norm T={T} d={d} {dtype} weighted={weighted}", flush=True)
    gen = torch.Generator().manual_seed(T * 7919 + d)
    x = (torch.randn(T, d, generator=gen) * 3.0).to(dtype)
    w = (1.0 + 0.1 * torch.randn(d, generator=gen)) if weighted else None
    eps = 1e-6
    xf = x.float()
    ref = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    if w is not None:
        ref = ref * w
    got = be().rms_norm(x.to(DEV), None if w is None else w.to(DEV), eps).cpu()
    assert got.dtype == dtype and got.shape == x.shape
    if T == 0:
        return
    if dtype == torch.bfloat16:
        exact = ref.to(torch.bfloat16)
        mism = (got != exact)
        assert float(mism.float().mean()) < 0.01
        # a mismatch is one bf16 ulp: the fp32 results sit next to a rounding boundary
        ulp = (exact.float().abs() * 2.0 ** -7).clamp_min(2.0 ** -133)
        assert bool(((got.float() - exact.float()).abs() <= ulp * 1.0001).all())
    else:
        assert rel_max(got, ref) < 4e-6
    with pytest.raises(ValueError):
        be().rms_norm(x.to(DEV), None, 0.0)


@pytest.mark.parametrize("T,d,h,E,k,dtype,weighted", [
    (64, 1024, 2560, 8, 2, torch.bfloat16, False),  # C4 layer: combine + norm in the down kernel's tail
    (64, 1024, 2560, 8, 2, torch.bfloat16, True),   # the same with a norm weight
    (20, 1024, 1024, 8, 2, torch.bfloat16, True),   # the same tail on the 2-block down instance
    (40, 2048, 256, 4, 2, torch.bfloat16, True),    # two chunks per lane
    (300, 256, 640, 8, 2, torch.bfloat16, True),    # prefill path
    (33, 192, 320, 4, 3, torch.float32, False),     # fp32 activations
    (300, 256, 640, 8, 2, torch.float32, True),     # fp32 activations on the hi / lo planes GEMMs
    (5, 4160, 128, 4, 2, torch.bfloat16, True),     # d > 4096: combine, then the norm kernel
])
def test_moe_forward_norm(T, d, h, E, k, dtype, weighted):
    """moe_forward_norm returns moe_forward's outputs unchanged plus
    rms_norm(out, weight, eps) bit for bit (the fused combine+norm sums the
    squares in rms_norm_kernel's order)."""
    print(f"case moe_forward_norm T={T} d={d} h={h} E={E} k={k} {dtype} weighted={weighted}", flush=True)
    x, gw, gb, experts = make_moe(T * 31 + d, T, d, h, E, k, dtype=dtype)
    gen = torch.Generator().manual_seed(d)
    w = (1.0 + 0.1 * torch.randn(d, generator=gen)).to(DEV) if weighted else None
    dx, dgw, dgb, dex = x.to(DEV), gw.to(DEV), gb.to(DEV), to_dev_experts(experts)
    ref = be().moe_forward(dx, dgw, dgb, dex, k, 64)
    got = be().moe_forward_norm(dx, dgw, dgb, dex, k, 64, w, 1e-6)
    normed = be().rms_norm(ref[0], w, 1e-6)
    torch.cuda.synchronize()
    for a, b in zip(ref, got[:4]):
        assert torch.equal(a.cpu(), b.cpu())
    assert torch.equal(got[4].cpu(), normed.cpu())
    # and the norm itself against the fp32 formula
    xf = ref[0].float().cpu()
    r = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    if w is not None:
        r = r * w.cpu()
    assert rel_max(got[4].float(), r) < (8e-3 if dtype == torch.bfloat16 else 4e-6)


@pytest.mark.parametrize("T,d,h,E,k,nE,nk,dtype", [
    (64, 1024, 2560, 8, 2, 8, 2, torch.bfloat16),   # C4 layer: decode path, router fused into the combine
    (40, 2048, 256, 4, 2, 16, 4, torch.bfloat16),   # two chunks per lane, 16 next experts
    (300, 256, 640, 8, 2, 6, 2, torch.bfloat16),    # prefill path, ragged last 16-token block, E < EMAX
    (33, 192, 320, 4, 3, 4, 3, torch.float32),      # fp32: the next router runs as its own kernel
    (300, 256, 640, 8, 2, 6, 2, torch.float32),     # fp32 on the hi / lo planes GEMMs, then norm and router
    (5, 4160, 128, 4, 2, 4, 2, torch.bfloat16),     # d > 4096: combine, norm, router kernels
    (7, 512, 384, 4, 2, 8, 3, torch.bfloat16),      # one partial 16-token block, fused router
    (20, 1024, 1024, 8, 2, 16, 4, torch.bfloat16),  # combine in the down kernel's tail: 3 workgroups, 16 experts
    (64, 512, 2560, 16, 2, 6, 2, torch.bfloat16),   # the same with 6 of 8 router lanes (not exact)
])
def test_moe_forward_chain(T, d, h, E, k, nE, nk, dtype):
    """Two chained layers: layer A routes its normalised output with layer B's
    router (next_router), layer B takes that routing (routing=).  Every output
    equals the unchained calls bit for bit: A's outputs those of
    moe_forward_norm, the next routing moe_router(normed), B's outputs those
    of moe_forward_norm on A's normalised output."""
    print(f"case moe_forward_chain T={T} d={d} h={h} E={E} k={k} nE={nE} nk={nk} {dtype}", flush=True)
    x, gwa, gba, exa = make_moe(T * 37 + d, T, d, h, E, k, dtype=dtype)
    _, gwb, gbb, exb = make_moe(T * 41 + h, 1, d, h, nE, nk, dtype=dtype)
    gen = torch.Generator().manual_seed(d + 1)
    w = (1.0 + 0.1 * torch.randn(d, generator=gen)).to(DEV)
    dx = x.to(DEV)
    dgwa, dgba, dexa = gwa.to(DEV), gba.to(DEV), to_dev_experts(exa)
    dgwb, dgbb, dexb = gwb.to(DEV), gbb.to(DEV), to_dev_experts(exb)
    ref_a = be().moe_forward_norm(dx, dgwa, dgba, dexa, k, 64, w, 1e-6)
    got_a = be().moe_forward_norm(dx, dgwa, dgba, dexa, k, 64, w, 1e-6, next_router=(dgwb, dgbb, nk))
    ref_r = be().moe_router(ref_a[4], dgwb, dgbb, nk)
    torch.cuda.synchronize()
    for a, b in zip(ref_a, got_a[:5]):
        assert torch.equal(a.cpu(), b.cpu())
    assert len(got_a) == 6
    for a, b in zip(ref_r, got_a[5]):
        assert torch.equal(a.cpu(), b.cpu())
    ref_b = be().moe_forward_norm(got_a[4], dgwb, dgbb, dexb, nk, 64, w, 1e-6)
    got_b = be().moe_forward_norm(got_a[4], dgwb, dgbb, dexb, nk, 64, w, 1e-6, routing=got_a[5])
    torch.cuda.synchronize()
    assert len(got_b) == 5
    for a, b in zip(ref_b, got_b):
        assert torch.equal(a.cpu(), b.cpu())


@pytest.mark.parametrize("T,h,nE", [(64, 2560, 8), (17, 1024, 16)])
def test_moe_chain_repeated(T, h, nE):
    """The decode layer whose combine tail waits on a workspace counter
    (cleared by the gate/up kernel of each call): 12 chained calls in a row,
    each equal bit for bit to the unchained layer and router."""
    d, E, k, nk = 1024, 8, 2, 2
    print(f"case chain repeated T={T} h={h} nE={nE}", flush=True)
    x, gw, gb, ex = make_moe(T * 7 + h, T, d, h, E, k, dtype=torch.bfloat16)
    _, gwb, gbb, _ = make_moe(T * 11 + nE, 1, d, h, nE, nk, dtype=torch.bfloat16)
    dx, dgw, dgb, dex = x.to(DEV), gw.to(DEV), gb.to(DEV), to_dev_experts(ex)
    dgwb, dgbb = gwb.to(DEV), gbb.to(DEV)
    ref = be().moe_forward_norm(dx, dgw, dgb, dex, k, 64, None, 1e-6)
    ref_r = be().moe_router(ref[4], dgwb, dgbb, nk)
    for it in range(12):
        got = be().moe_forward_norm(dx, dgw, dgb, dex, k, 64, None, 1e-6, next_router=(dgwb, dgbb, nk))
        torch.cuda.synchronize()
        for a, b in zip(ref, got[:5]):
            assert torch.equal(a.cpu(), b.cpu()), it
        for a, b in zip(ref_r, got[5]):
            assert torch.equal(a.cpu(), b.cpu()), it


@pytest.mark.parametrize("mode", ["chain", "norm", "plain"])
def test_decode_tail_wait_give_up_is_loud(mode):
    """The decode combine in the down kernel's tail waits (bounded) for every
    workgroup of the launch.  Forced from the host to give up -- the test hook
    asks for one arrival more than the grid holds and allows 64 polls, so
    every kernel still exits normally -- each combining workgroup must poison
    its tokens (NaN out / norm_out rows, NaN next prob / topw, next topi -1)
    instead of combining, and count itself in smaul_wait_timeouts.  The
    layer's own routing and counts are unaffected, and the next call with the
    default wait is whole again."""
    from smaulnative_amd import _lib
    lib = _lib.load()
    T, d, h, E, k = 64, 1024, 2560, 8, 2
    print(f"case tail wait give-up mode={mode} T={T}", flush=True)
    x, gw, gb, ex = make_moe(4242, T, d, h, E, k, dtype=torch.bfloat16)
    _, gwb, gbb, _ = make_moe(4243, 1, d, h, E, k, dtype=torch.bfloat16)
    dx, dgw, dgb, dex = x.to(DEV), gw.to(DEV), gb.to(DEV), to_dev_experts(ex)
    nxt = (gwb.to(DEV), gbb.to(DEV), k)

    def call():
        if mode == "chain":
            return be().moe_forward_norm(dx, dgw, dgb, dex, k, 64, None, 1e-6, next_router=nxt)
        if mode == "norm":
            return be().moe_forward_norm(dx, dgw, dgb, dex, k, 64, None, 1e-6)
        return be().moe_forward(dx, dgw, dgb, dex, k, 64)

    be().wait_timeouts(DEV, reset=True)
    ref = call()
    assert be().wait_timeouts(DEV) == 0
    _lib.check(lib.smaul_debug_tail_wait(1, 64), "debug_tail_wait")
    try:
        got = call()
        torch.cuda.synchronize()
    finally:
        _lib.check(lib.smaul_debug_tail_wait(0, 1 << 20), "debug_tail_wait")
    # ceil(T / 8) combining workgroups, each gave up once
    assert be().wait_timeouts(DEV, reset=True) == (T + 7) // 8
    assert torch.isnan(got[0].float()).all()
    for a, b in zip(ref[1:4], got[1:4]):  # prob, topi, counts of this layer
        assert torch.equal(a.cpu(), b.cpu())
    if mode != "plain":
        assert torch.isnan(got[4].float()).all()
    if mode == "chain":
        nprob, ntopi, ntopw = got[5]
        assert torch.isnan(nprob).all() and torch.isnan(ntopw).all()
        assert (ntopi == -1).all()
    again = call()
    torch.cuda.synchronize()
    assert be().wait_timeouts(DEV) == 0
    flat = lambda r: [t for v in r for t in (v if isinstance(v, tuple) else (v,))]
    for a, b in zip(flat(ref), flat(again)):
        assert torch.equal(a.cpu(), b.cpu())
