"""smaulnative_amd -- MI355X-native tiled-FP8 MoE forward for SmaulNative.

Public surface (mirrors the reference's names):
- ``compute.get_backend`` / ``compute.register_backend`` and the ``rocm``
  backend (``rocm_backend.RocmBackend``);
- ``fp8_tile.FP8Linear``, ``fp8_tile.quantize_tiles``, ``fp8_tile.decode_tile``;
- ``moe.SwiFFN``, ``moe.SwiFFN_MoE``.
The compute itself is libsmaul_rocm.so (HIP for gfx950, C ABI in
include/smaul_rocm.h).
"""
from smaulnative_amd.compute import get_backend, register_backend  # noqa: F401
from smaulnative_amd.fp8_tile import FP8Linear, quantize_tiles, decode_tile  # noqa: F401
from smaulnative_amd.moe import MoEConfig, SwiFFN, SwiFFN_MoE  # noqa: F401

__version__ = "0.1.0"
