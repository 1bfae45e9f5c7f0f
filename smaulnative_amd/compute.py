"""Compute-backend registry, the same boundary as the reference's kernel/compute.py.

Reference: kernel/compute.py:48-61 (``_BACKENDS``, ``register_backend``,
``get_backend``).  The model code calls ``get_backend()`` and never touches an
extension directly; backends register themselves by ``name``.  Unknown names
raise ``ValueError`` listing what is registered -- there are no fake
backends.

This package registers exactly one backend, ``"rocm"`` (``RocmBackend``), so
the default selection (environment variable ``SMAUL_BACKEND``) is ``"rocm"``.
In the reference checkout the same object is registered next to the CPU
backend and selected with ``SMAUL_BACKEND=rocm``.
"""
from __future__ import annotations

import os

_BACKENDS: dict = {}
DEFAULT_BACKEND = "rocm"


def register_backend(backend):
    """compute.py:51-53: key the backend object by its ``name``."""
    _BACKENDS[backend.name] = backend
    return backend


def get_backend(name=None):
    """compute.py:56-61: ``name`` or $SMAUL_BACKEND, else the default."""
    name = name or os.environ.get("SMAUL_BACKEND", DEFAULT_BACKEND)
    try:
        return _BACKENDS[name]
    except KeyError:
        raise ValueError(f"unknown compute backend {name!r}; registered: {sorted(_BACKENDS)}") from None


def registered():
    return sorted(_BACKENDS)


from smaulnative_amd.rocm_backend import RocmBackend  # noqa: E402

register_backend(RocmBackend())
