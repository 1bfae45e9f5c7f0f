"""smaul_moe_forward_noalloc (static scratch, no allocation) against smaul_moe_forward.

Both run the same kernels; the only difference is where the layer's workspace
lives (a static device array inside the library instead of a caller
workspace), so every output must be bit-identical.  Two calls in a row, the
second with a smaller input, check that nothing left in the shared array by
the first call leaks into the second.
"""
import pytest
import torch

import oracle
from smaulnative_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _layer(seed, T, d, h, E, k):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(T, d, generator=gen).to(torch.bfloat16)
    gw = torch.randn(E, d, generator=gen) * 0.02
    gb = torch.randn(E, generator=gen) * 0.5
    experts = [oracle.make_expert(d, h, gen) for _ in range(E)]
    return x, gw, gb, experts


def _run(lib, noalloc, x, gw, gb, experts, k):
    T, d = x.shape
    E = len(experts)
    h = experts[0].gate_w.shape[0]
    bufs = [[t.to(DEV) for t in (ex.gate_w, ex.gate_s, ex.up_w, ex.up_s, ex.down_w, ex.down_s)] for ex in experts]
    table = torch.tensor([[b[j].data_ptr() for b in bufs] for j in range(6)], dtype=torch.int64, device=DEV)
    xd, gwd, gbd = x.to(DEV), gw.to(DEV), gb.to(DEV)
    out = torch.empty_like(xd)
    prob = torch.empty(T, E, device=DEV)
    topi = torch.empty(T, k, dtype=torch.int64, device=DEV)
    topw = torch.empty(T, k, device=DEV)
    counts = torch.empty(E, dtype=torch.int32, device=DEV)
    tp, row = table.data_ptr(), E * 8
    ptrs = [tp + j * row for j in range(6)]
    stream = torch.cuda.current_stream().cuda_stream
    head = [xd.data_ptr(), _lib.DTYPE_BF16, gwd.data_ptr(), gbd.data_ptr(), *ptrs, out.data_ptr(),
            prob.data_ptr(), topi.data_ptr(), topw.data_ptr(), counts.data_ptr()]
    if noalloc:
        rc = lib.smaul_moe_forward_noalloc(*head, T, d, h, E, k, 64, _lib.FLAG_ALIGNED_CODES, stream)
        ws = None
    else:
        ws_bytes = lib.smaul_moe_workspace_size(T, d, h, E, k, _lib.DTYPE_BF16)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
        rc = lib.smaul_moe_forward(*head, ws.data_ptr(), ws_bytes, T, d, h, E, k, 64, _lib.FLAG_ALIGNED_CODES, stream)
    _lib.check(rc, "noalloc" if noalloc else "moe_forward")
    torch.cuda.synchronize()
    del ws, bufs, table
    return [t.cpu() for t in (out, prob, topi, topw, counts)]


def test_noalloc_matches_workspace_entry_two_calls():
    lib = _lib.load()
    # first a prefill-sized layer (dispatch kernels, 128-row tiles), then a
    # smaller decode-sized one (decode kernels) that reuses the same array
    for seed, T, d, h, E, k in ((1, 1200, 1024, 2560, 8, 2), (2, 64, 1024, 2560, 8, 2)):
        print(f"case noalloc T={T} d={d} h={h} E={E} k={k}", flush=True)
        x, gw, gb, experts = _layer(seed, T, d, h, E, k)
        ref = _run(lib, False, x, gw, gb, experts, k)
        got = _run(lib, True, x, gw, gb, experts, k)
        for a, b in zip(ref, got):
            assert torch.equal(a, b)
        o = oracle.moe_forward(x, gw, gb, experts, k)
        assert torch.equal(got[2], o.topi)
        err = float((got[0].double() - o.out.double()).norm() / o.out.double().norm())
        assert err < 2e-3, err


def test_noalloc_rejects_layers_beyond_the_scratch():
    lib = _lib.load()
    T, d, h, E, k = 16384, 1024, 2560, 8, 2
    assert lib.smaul_moe_workspace_size(T, d, h, E, k, _lib.DTYPE_BF16) > (64 << 20)
    rc = lib.smaul_moe_forward_noalloc(*([None, _lib.DTYPE_BF16] + [None] * 13), T, d, h, E, k, 64, 0, None)
    assert rc == _lib.SMAUL_ERR_UNSUPPORTED and "static" in _lib.last_error()
