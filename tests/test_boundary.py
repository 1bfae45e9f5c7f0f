"""CPU checks of the drop-in boundary: the C-ABI library and the Python backend surface.

No compute call reaches a GPU here; these cover the library's exports, the
host-side top-k order, argument validation and the no-fallback rule.
"""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from smaulnative_amd import _lib
from smaulnative_amd.compute import get_backend, register_backend, registered

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "smaul_rocm.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(smaul_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    names = declared_symbols()
    assert len(names) >= 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers the same set
    assert sorted(_lib.SIGNATURES) == names


def test_library_version_and_error_channel():
    lib = _lib.load()
    assert lib.smaul_version() >= 100
    assert isinstance(_lib.last_error(), str)


def test_library_validates_without_touching_the_gpu():
    lib = _lib.load()
    # non-positive sizes are rejected before any launch
    rc = lib.smaul_fp8_linear(None, 0, None, None, None, 0, 4, 0, 8, 64, 0, None)
    assert rc == _lib.SMAUL_ERR_INVALID and "positive" in _lib.last_error()
    rc = lib.smaul_fp8_linear(None, 0, None, None, None, 0, 4, 64, 8, 48, 0, None)
    assert rc == _lib.SMAUL_ERR_UNSUPPORTED
    # the workspace entry reports what smaul_fp8_linear reports
    rc = lib.smaul_fp8_linear_ws(None, 0, None, None, None, 0, 4, 0, 8, 64, 0, None, 0, None)
    assert rc == _lib.SMAUL_ERR_INVALID and "positive" in _lib.last_error()
    rc = lib.smaul_fp8_linear_ws(None, 0, None, None, None, 0, 4, 64, 8, 48, 0, None, 0, None)
    assert rc == _lib.SMAUL_ERR_UNSUPPORTED
    assert lib.smaul_fp8_linear_workspace_size(2000, 512, 0) == 2000 * 512 * 4
    assert lib.smaul_fp8_linear_workspace_size(100, 512, 0) == 0
    assert lib.smaul_fp8_linear_workspace_size(100, 512, 1) == 0
    rc = lib.smaul_moe_router(None, 1, None, None, None, None, None, 8, 64, 65, 2, None)
    assert rc == _lib.SMAUL_ERR_INVALID
    assert lib.smaul_moe_workspace_size(16384, 1024, 2560, 8, 2, 1) > 2 * 32768 * 2560
    # RMSNorm: eps must be positive and finite (model.py:127-128), dtype known
    rc = lib.smaul_rms_norm(None, 1, None, None, 4, 64, 0.0, None)
    assert rc == _lib.SMAUL_ERR_INVALID and "eps" in _lib.last_error()
    rc = lib.smaul_rms_norm(None, 7, None, None, 4, 64, 1e-6, None)
    assert rc == _lib.SMAUL_ERR_INVALID
    assert lib.smaul_rms_norm(None, 1, None, None, 0, 64, 1e-6, None) == _lib.SMAUL_OK  # nothing to do
    rc = lib.smaul_moe_forward_norm(None, 1, None, None, None, None, None, None, None, None, None, None, None,
                                    None, None, None, 0, 64, 64, 128, 8, 2, 64, 0, None, float("nan"), None, None)
    assert rc == _lib.SMAUL_ERR_INVALID and "eps" in _lib.last_error()
    # the chained layer: eps, a routed call without its routing, the next router's sizes
    head = [None, 1, None, None, None, None, None, None, None, None, None, None, None, None, None, None]
    rc = lib.smaul_moe_forward_chain(*head, 0, 4, 64, 128, 8, 2, 64, 0, None, 0.0, None, 0,
                                     None, None, 0, 0, None, None, None, None)
    assert rc == _lib.SMAUL_ERR_INVALID and "eps" in _lib.last_error()
    rc = lib.smaul_moe_forward_chain(*head, 0, 4, 64, 128, 8, 2, 64, 0, None, 1e-6, 16, 1,
                                     None, None, 0, 0, None, None, None, None)
    assert rc == _lib.SMAUL_ERR_INVALID and "routed" in _lib.last_error()
    rc = lib.smaul_moe_forward_chain(*head, 0, 4, 64, 128, 8, 2, 64, 0, None, 1e-6, 16, 0,
                                     16, None, 65, 2, None, None, None, None)
    assert rc == _lib.SMAUL_ERR_INVALID and "router" in _lib.last_error()
    # the tiled relayout: K % 64, and outputs that overlap their inputs (the
    # addresses are never dereferenced: the checks come before any launch)
    a, b = 1 << 32, 1 << 33
    assert lib.smaul_fp8_tile_layout(a, b, a + (1 << 20), b + (1 << 20), 4, 96, None) == _lib.SMAUL_ERR_INVALID
    assert "multiple of 64" in _lib.last_error()
    N, K = 8, 128
    for co, so in ((a, b + (1 << 20)), (a + 512, b + (1 << 20)), (a + (1 << 20), b + 4)):
        rc = lib.smaul_fp8_tile_layout(a, b, co, so, N, K, None)
        assert rc == _lib.SMAUL_ERR_INVALID and "overlap" in _lib.last_error()


def _host_topk(vals, k):
    lib = _lib.load()
    v = np.ascontiguousarray(vals, dtype=np.float32)
    out = np.zeros(k, dtype=np.int64)
    assert lib.smaul_selftest_topk(v.ctypes.data, v.size, k, out.ctypes.data) == 0
    return out


def test_router_topk_order_matches_torch_on_ties():
    gen = torch.Generator().manual_seed(0)
    for trial in range(3000):
        n = int(torch.randint(1, 65, (1,), generator=gen))
        k = int(torch.randint(1, n + 1, (1,), generator=gen))
        if trial % 5 == 0:
            n, k = 64, 1  # torch's partial_sort branch (k * 64 <= n)
        mode = trial % 4
        if mode == 0:
            v = torch.randint(0, 3, (n,), generator=gen).float()
        elif mode == 1:
            v = torch.full((n,), 0.125)
        elif mode == 2:
            v = torch.rand(n, generator=gen)
        else:
            v = torch.randint(0, 4, (n,), generator=gen).float()
            v[torch.rand(n, generator=gen) < 0.1] = float("nan")
        ref = torch.topk(v, k, -1)[1].numpy()
        assert np.array_equal(_host_topk(v.numpy(), k), ref), (n, k, v.tolist())


def test_registry_contract():
    be = get_backend()
    assert be.name == "rocm" and "rocm" in registered()
    with pytest.raises(ValueError, match="unknown compute backend"):
        get_backend("cpu-fake")

    class Other:
        name = "other-test"
    register_backend(Other())
    assert get_backend("other-test").name == "other-test"


def test_backend_surface_and_no_fallback():
    be = get_backend("rocm")
    for attr in ("configure", "fp8_forward", "fp8_backward_input", "fp8_quantize_tiles",
                 "attn_forward", "attn_step", "attn_backward", "sparse_grad_v", "moe_forward"):
        assert callable(getattr(be, attr)), attr
    assert be.has_native is True
    assert be.has_attn_native is True and be.has_sparse_native is False
    assert be.configure(2) == 2
    w = torch.zeros(8, 64, dtype=torch.uint8)
    s = torch.ones(8, 1)
    with pytest.raises(ValueError):
        be.fp8_forward(torch.zeros(2, 64), w, s, 64, 8, 0)
    with pytest.raises(RuntimeError, match="HIP device"):
        be.fp8_forward(torch.zeros(2, 64), w, s, 64, 8, 64)  # CPU tensors: raise, never fall back
    with pytest.raises(RuntimeError, match="HIP device"):
        be.fp8_backward_input(torch.zeros(2, 8), w, s, 64, 8, 64)  # the device backward, no host fallback
    q = torch.zeros(1, 2, 1, 8)
    with pytest.raises(RuntimeError, match="HIP device"):
        be.attn_backward(q, q, q, q, q, torch.ones(1, 2, 1), 1e-6)  # the device backward, no host fallback
    with pytest.raises(NotImplementedError):
        be.sparse_grad_v(None, None, None, None)
    assert be.fp8_quantize_tiles(torch.zeros(8, 64), 64) is None


def test_fp8linear_and_moe_modules_on_cpu():
    from smaulnative_amd import FP8Linear, MoEConfig, SwiFFN_MoE
    m = FP8Linear(100, 40, 64)
    assert m.w8.dtype == torch.uint8 and tuple(m.w8.shape) == (40, 100)
    assert tuple(m.sc.shape) == (40, 2) and m.sc.dtype == torch.float32
    with pytest.raises(RuntimeError, match="HIP device"):
        m(torch.randn(3, 100))
    with pytest.raises(ValueError):
        SwiFFN_MoE(MoEConfig(d_model=64, num_experts=2, num_experts_per_tok=3))
    moe = SwiFFN_MoE(MoEConfig(d_model=64, num_experts=4, num_experts_per_tok=2))
    assert len(moe.experts) == 4 and moe.experts[0].gate.out_f == 160
    assert moe.routing_stats()["token_counts"] == [0, 0, 0, 0]
    with torch.no_grad(), pytest.raises(RuntimeError, match="HIP device"):
        moe(torch.randn(1, 4, 64))
    aux = moe.balance_loss(torch.full((8, 4), 0.25))
    assert abs(float(aux) - 1.0) < 1e-6


def test_staged_entries_need_device_tensors():
    """Every backend entry that hands pointers to the library checks that its
    tensors live on a HIP device first: a host pointer never reaches a kernel."""
    be = get_backend("rocm")
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    gw = torch.zeros(4, 64)
    with pytest.raises(RuntimeError, match="HIP device"):
        be.moe_router(x, gw, None, 2)
    with pytest.raises(RuntimeError, match="HIP device"):
        be.moe_dispatch(torch.zeros(4, 2, dtype=torch.int64), torch.zeros(4, 2), 4)
    with pytest.raises(RuntimeError, match="HIP device"):
        be.moe_stages(x, gw, None, [()] * 4, 2, 64)
    with pytest.raises(RuntimeError, match="HIP device"):
        be.moe_forward(x, gw, torch.zeros(4), [()] * 4, 2, 64)
