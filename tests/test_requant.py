"""The FP8Linear weight updates against the reference's own outputs (CPU).

requant / fused_lion_requant (kernel/fp8_tile.py:240-285) replayed on the
inputs of tests/golden/golden_requant.npz, which make_golden_requant.py wrote
by running the reference's FP8Linear: codes, scales and Lion momentum must be
bit-identical.  Host tensors take the torch quantizer path (the backend
contract's None, kernel/compute.py:246-263); the GPU test replays the same
cases on device buffers.
"""
import os

import numpy as np
import pytest
import torch

from smaulnative_amd.fp8_tile import FP8Linear, decode_block, decode_tile

GOLD = os.path.join(os.path.dirname(__file__), "golden", "golden_requant.npz")


def _t(a):
    a = np.array(a)
    return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16) if a.dtype == np.int16 else torch.from_numpy(a)


def _module(g, key, tile, device):
    w8, sc = _t(g[f"{key}_w8"]), _t(g[f"{key}_sc"])
    out_f, in_f = w8.shape
    m = FP8Linear(in_f, out_f, tile)
    m.w8.copy_(w8)
    m.sc.copy_(sc)
    return m.to(device)


def replay(device):
    """Every case of the fixture on `device`; asserts bit equality."""
    g = np.load(GOLD)
    for name in ("a", "b", "c"):
        in_f, out_f, tile, decay = g[f"rq_{name}_meta"]
        m = _module(g, f"rq_{name}", int(tile), device)
        m.requant(_t(g[f"rq_{name}_upd"]).to(device), float(decay))
        assert torch.equal(m.w8.cpu(), _t(g[f"rq_{name}_w8_out"])), name
        assert torch.equal(m.sc.cpu(), _t(g[f"rq_{name}_sc_out"])), name
    m = _module(g, "rq_none", 64, device)
    m.requant(None, 0.0)
    assert torch.equal(m.w8.cpu(), _t(g["rq_none_w8_out"]))
    assert torch.equal(m.sc.cpu(), _t(g["rq_none_sc_out"]))
    lr, wd, b1, b2 = (float(v) for v in g["lion_meta"])
    m = _module(g, "lion", 32, device)
    gw, st = _t(g["lion_gw"]).to(device), _t(g["lion_st"]).clone().to(device)
    gw0 = gw.clone()
    m._gw = gw
    m.fused_lion_requant(gw, st, lr, wd, b1, b2)
    assert m._gw is None and torch.equal(gw, gw0)
    assert torch.equal(st.cpu(), _t(g["lion_st_out"]))
    assert torch.equal(m.w8.cpu(), _t(g["lion_w8_out"]))
    assert torch.equal(m.sc.cpu(), _t(g["lion_sc_out"]))


def test_requant_and_lion_match_reference_cpu():
    replay("cpu")


def test_requant_rejects_transposed_update():
    m = FP8Linear(64, 32, 64)
    with pytest.raises(ValueError, match="transposed"):
        m.requant(torch.zeros(64, 32))


def test_decode_block_is_the_per_tile_decode():
    m = FP8Linear(100, 19, 32)
    blk = decode_block(m.w8, m.sc, 2, 17, 100, 32)
    ref = torch.cat([decode_tile(m.w8, m.sc, 2, 17, t, 32) for t in range(4)], 1)
    assert torch.equal(blk, ref)


def test_err_stats():
    m = FP8Linear(128, 16, 64)
    st = m.err_stats()
    full = decode_block(m.w8, m.sc, 0, 16, 128, 64)
    assert st["amax_fp8"] == float(full.abs().max())
    assert abs(st["mean_scale"] - float(m.sc.double().mean())) == 0.0
