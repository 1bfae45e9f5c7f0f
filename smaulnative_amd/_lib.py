"""ctypes binding of libsmaul_rocm.so (the C ABI declared in include/smaul_rocm.h).

The library is built in-tree by ``smaulnative_amd.build`` (hipcc, gfx950) and
loaded from the package directory.  There is no other implementation: if the
library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsmaul_rocm.so")

SMAUL_OK = 0
SMAUL_ERR_INVALID = 1
SMAUL_ERR_UNSUPPORTED = 2
SMAUL_ERR_HIP = 3
DTYPE_F32 = 0
DTYPE_BF16 = 1
FLAG_CANONICAL_CODES = 1
FLAG_ALIGNED_CODES = 2
FLAG_TILED_LAYOUT = 4

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int

# name -> (restype, argtypes); mirrors include/smaul_rocm.h one to one.
SIGNATURES = {
    "smaul_version": (_I, []),
    "smaul_last_error": (ctypes.c_char_p, []),
    "smaul_fp8_linear": (_I, [_P, _I, _P, _P, _P, _I, _I64, _I64, _I64, _I64, _I, _P]),
    "smaul_fp8_linear_workspace_size": (_I64, [_I64, _I64, _I]),
    "smaul_fp8_linear_ws": (_I, [_P, _I, _P, _P, _P, _I, _I64, _I64, _I64, _I64, _I, _P, _I64, _P]),
    "smaul_fp8_canonicalize": (_I, [_P, _P, _I64, _P]),
    "smaul_fp8_tile_layout": (_I, [_P, _P, _P, _P, _I64, _I64, _P]),
    "smaul_moe_router": (_I, [_P, _I, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "smaul_moe_dispatch_workspace_size": (_I64, [_I64, _I64]),
    "smaul_moe_dispatch": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P]),
    "smaul_moe_block_m": (_I, [_I64, _I64, _I64, _I64, _I64, _I64, _I]),
    "smaul_moe_gate_up": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                               _I64, _I64, _I, _P]),
    "smaul_moe_down": (_I, [_P, _I, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P]),
    "smaul_moe_combine": (_I, [_P, _I, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "smaul_rms_norm": (_I, [_P, _I, _P, _P, _I64, _I64, ctypes.c_float, _P]),
    "smaul_moe_workspace_size": (_I64, [_I64, _I64, _I64, _I64, _I64, _I]),
    "smaul_moe_forward": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                               _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P]),
    "smaul_moe_forward_noalloc": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                       _I64, _I64, _I64, _I64, _I64, _I64, _I, _P]),
    "smaul_moe_forward_norm": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                    _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P, ctypes.c_float, _P, _P]),
    "smaul_moe_forward_chain": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                     _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P, ctypes.c_float, _P, _I,
                                     _P, _P, _I64, _I64, _P, _P, _P, _P]),
    "smaul_swiffn_workspace_size": (_I64, [_I64, _I64, _I]),
    "smaul_swiffn_forward": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _P]),
    "smaul_attn_workspace_size": (_I64, [_I64, _I64, _I64, _I]),
    "smaul_attn_forward": (_I, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, ctypes.c_float, _P, _I64, _P]),
    "smaul_attn_step": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, ctypes.c_float, _P]),
    "smaul_attn_backward": (_I, [_P] * 9 + [_I64, _I64, _I64, _I64, ctypes.c_float, _P, _I64, _P]),
    "smaul_fp8_quantize_tiles": (_I, [_P, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _P, _P]),
    "smaul_fp8_backward_input": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "smaul_wait_timeouts": (_I, [_P, _I, _P]),
    "smaul_debug_tail_wait": (_I, [_I, _I]),
    "smaul_peak_mfma": (_I, [_P, _I, _I, _P]),
    "smaul_peak_stream": (_I, [_P, _I64, _P, _I, _P]),
    "smaul_peak_lds_dma": (_I, [_P, _I64, _P, _I, _I, _P]),
    "smaul_selftest_topk": (_I, [_P, _I64, _I64, _P]),
}

_lib = None
_lock = threading.Lock()


class LibraryMissing(RuntimeError):
    pass


def load():
    """Load (once) and return the ctypes library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise LibraryMissing(
                    f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                    "or `python -m smaulnative_amd.build`")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def last_error() -> str:
    msg = load().smaul_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(rc: int, what: str) -> None:
    """Map a library status to a Python exception."""
    if rc == SMAUL_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc == SMAUL_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    if rc == SMAUL_ERR_INVALID:
        raise ValueError(msg)
    raise RuntimeError(msg)
