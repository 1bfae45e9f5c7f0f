"""The ``rocm`` compute backend: the reference backend surface on MI355X.

Reference surface (kernel/compute.py:64-322, every call site in the reference):
``name``, ``configure``, ``has_native`` / ``has_attn_native`` /
``has_sparse_native``, ``fp8_forward``, ``fp8_backward_input``,
``fp8_quantize_tiles``, ``attn_forward`` / ``attn_step`` / ``attn_backward``,
``sparse_grad_v``.  This backend adds ``moe_forward`` (and its stages), the
entry the MoE layer calls; the reference has no MoE hook because its routing
is plain torch code inside SwiFFN_MoE.forward (model.py:557-585).

Behaviour differences from the reference CPU backend, all deliberate:
- nothing falls back: where the reference warns once and runs a torch
  fallback (compute.py:134,137-143), this backend raises;
- inputs must be HIP device tensors; work is enqueued on the current stream
  and nothing synchronises;
- ``fp8_forward`` also accepts bf16 ``x`` (fed to bf16 MFMA unchanged);
  fp32 ``x`` is split into two bf16 terms inside the kernel;
- ``attn_forward`` / ``attn_step`` run the linear-attention recurrence on the
  device, bit-identical to the reference's native kernels (attn_cpu.cpp);
- ``fp8_quantize_tiles`` quantizes HIP tensors on the device (bit-identical
  codes and scales); for host tensors it returns ``None``, which the contract
  defines as "run the torch quantizer" (compute.py:246-263, fp8_tile.py:96-113);
- ``fp8_backward_input`` (the FP8Linear input gradient) and ``attn_backward``
  (the recurrence's two-pass backward, bit-identical to attn_cpu.cpp) run on
  the device; ``sparse_grad_v`` (Rawr) is not built and raises
  ``NotImplementedError``.
"""
from __future__ import annotations

import math
import os
import threading
import weakref
from typing import Sequence

import torch

from smaulnative_amd import _lib

_ACT = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16}


def _stream_handle(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class _CacheEntry(dict):
    """One expert-cache entry (a dict that can be weakly referenced)."""


def _drop_entry(backend_ref, key, entry_ref):
    """Finalizer of a source buffer: evict its cache entry if both still live.
    It holds only weak references, so it keeps neither alive."""
    be, ent = backend_ref(), entry_ref()
    if be is not None and ent is not None:
        be._evict(key, ent)


def _need_device(name: str, *tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{name}: rocm backend needs HIP device tensors, got {t.device}")
    dev = tensors[0].device
    for t in tensors[1:]:
        if t is not None and t.device != dev:
            raise RuntimeError(f"{name}: tensors are on different devices ({dev} vs {t.device})")


class RocmBackend:
    """MI355X backend over libsmaul_rocm.so (hand-written HIP for gfx950)."""

    name = "rocm"

    def __init__(self):
        self._lock = threading.Lock()
        self._ptr_cache: dict = {}

    # ---- compute.py:77-103 ------------------------------------------------
    @staticmethod
    def _resolve_threads(threads):
        """An explicit count wins, then SMAUL_CPU_THREADS, then half the host's cores
        (at least one); a value that is not a number raises ValueError."""
        env = os.environ.get("SMAUL_CPU_THREADS")
        if threads is None and env:
            source, threads, parse = "SMAUL_CPU_THREADS", env, lambda v: int(float(v))  # "4.0" is accepted
        else:
            source, parse = "threads", int
        if threads is None:
            return max(1, (os.cpu_count() or 2) // 2)
        try:
            n = parse(threads)
        except (TypeError, ValueError):
            raise ValueError(f"{source}: expected a whole number of threads, got {threads!r}") from None
        return max(1, n)

    def configure(self, threads=None):
        """Set the host thread count for torch's CPU-side work and return it.

        The device path does not use host threads; this keeps the backend
        interface whole (train.py and benchmark.py call it).  OMP/MKL variables
        are overwritten, not defaulted, so an explicit count beats a stale
        exported value for native code loaded afterwards.
        """
        n = self._resolve_threads(threads)
        for var in ("OMP_NUM_THREADS", "MKL_NUM_THREADS"):
            os.environ[var] = str(n)
        torch.set_num_threads(n)
        try:
            torch.set_num_interop_threads(1)
        except RuntimeError:  # already fixed once torch has run parallel work
            pass
        return n

    @property
    def has_native(self):
        try:
            _lib.load()
            return True
        except _lib.LibraryMissing:
            return False

    @property
    def has_attn_native(self):
        return self.has_native

    @property
    def has_sparse_native(self):
        return False

    # ---- FP8 linear (compute.py:125-135, fp8_cpu.cpp:100-141) ---------------
    def fp8_forward(self, x, w, s, in_f, out_f, tile):
        """y[rows, out_f] fp32 = x[rows, in_f] . decode(w, s)^T on the HIP device."""
        if tile <= 0 or in_f <= 0 or out_f <= 0:
            raise ValueError(f"tile/in_f/out_f must be positive, got {tile}/{in_f}/{out_f}")
        lib = _lib.load()
        _need_device("fp8_forward", x, w, s)
        if x.dtype not in _ACT:
            raise RuntimeError(f"fp8_forward: x must be float32 or bfloat16, got {x.dtype}")
        if w.dtype != torch.uint8:
            raise RuntimeError(f"fp8_forward: w must be uint8, got {w.dtype}")
        if x.dim() != 2 or x.shape[1] != in_f:
            raise RuntimeError(f"fp8_forward: x must be [rows, in_f={in_f}], got {tuple(x.shape)}")
        nt = (in_f + tile - 1) // tile
        if w.numel() != out_f * in_f or s.numel() != out_f * nt:
            raise RuntimeError(f"fp8_forward: size mismatch w={w.numel()} s={s.numel()} expected "
                               f"{out_f * in_f} and {out_f * nt}")
        if not ((w.dim() == 2 and tuple(w.shape) == (out_f, in_f)) or w.dim() == 1):
            raise RuntimeError("fp8_forward: w must be [out_f, in_f] or flattened [out_f*in_f]")
        if not ((s.dim() == 2 and tuple(s.shape) == (out_f, nt)) or s.dim() == 1):
            raise RuntimeError("fp8_forward: s must be [out_f, nt] or flattened")
        xc = x if x.is_contiguous() else x.contiguous()
        wc = w.reshape(-1).contiguous()
        sc = s.reshape(-1)
        sc = (sc if sc.dtype == torch.float32 else sc.float()).contiguous()
        rows = xc.shape[0]
        y = torch.empty(rows, out_f, dtype=torch.float32, device=x.device)
        if rows == 0:
            return y
        # fp32 x (what FP8Linear passes) goes through a workspace of bf16 hi/lo
        # planes so the LDS-DMA GEMM can take it; bf16 x needs none
        nws = lib.smaul_fp8_linear_workspace_size(rows, in_f, _ACT[xc.dtype])
        ws = torch.empty(max(nws, 0), dtype=torch.uint8, device=x.device) if nws > 0 else None
        with torch.cuda.device(x.device):
            rc = lib.smaul_fp8_linear_ws(xc.data_ptr(), _ACT[xc.dtype], wc.data_ptr(), sc.data_ptr(),
                                         y.data_ptr(), _lib.DTYPE_F32, rows, in_f, out_f, tile, 0,
                                         None if ws is None else ws.data_ptr(), max(nws, 0),
                                         _stream_handle(x.device))
        _lib.check(rc, "fp8_forward")
        return y

    def fp8_backward_input(self, g, w, s, in_f, out_f, tile):
        """dx[rows, in_f] fp32 = g[rows, out_f] . decode(w, s) on the device
        (compute.py:145-153, fp8_cpu.cpp:167-259; fp32, another summation order)."""
        if tile <= 0 or in_f <= 0 or out_f <= 0:
            raise ValueError(f"tile/in_f/out_f must be positive, got {tile}/{in_f}/{out_f}")
        lib = _lib.load()
        _need_device("fp8_backward_input", g, w, s)
        if g.dtype != torch.float32 or w.dtype != torch.uint8:
            raise RuntimeError(f"fp8_backward_input: expected dtypes f32/u8, got {g.dtype}/{w.dtype}")
        if g.dim() != 2 or g.shape[1] != out_f:
            raise RuntimeError(f"fp8_backward_input: g must be [rows, out_f={out_f}], got {tuple(g.shape)}")
        nt = (in_f + tile - 1) // tile
        if w.numel() != out_f * in_f or s.numel() != out_f * nt:
            raise RuntimeError(f"fp8_backward_input: size mismatch w={w.numel()} s={s.numel()} expected "
                               f"{out_f * in_f} and {out_f * nt}")
        gc = g if g.is_contiguous() else g.contiguous()
        wc = w.reshape(-1).contiguous()
        sc = s.reshape(-1)
        sc = (sc if sc.dtype == torch.float32 else sc.float()).contiguous()
        dx = torch.empty(g.shape[0], in_f, dtype=torch.float32, device=g.device)
        with torch.cuda.device(g.device):
            rc = lib.smaul_fp8_backward_input(gc.data_ptr(), wc.data_ptr(), sc.data_ptr(), dx.data_ptr(), g.shape[0],
                                              in_f, out_f, tile, _stream_handle(g.device))
        _lib.check(rc, "fp8_backward_input")
        return dx

    def fp8_quantize_tiles(self, w32, tile):
        """(codes uint8 [out_f, nt*tile], scales fp32 [out_f, nt], non-finite count) on the device.

        compute.py:246-263 / quant_cpu.cpp:64-137, bit-identical codes and
        scales.  Host tensors return None, which the contract defines as
        "the caller runs the torch quantizer" (fp8_tile.py:96-113).
        """
        if not (isinstance(w32, torch.Tensor) and w32.is_cuda):
            return None
        if tile <= 0:
            raise ValueError(f"tile must be > 0, got {tile}")
        if w32.dim() != 2 or w32.dtype != torch.float32:
            raise RuntimeError(f"fp8_quantize_tiles: w32 must be 2-D float32, got {w32.dtype} dim {w32.dim()}")
        from smaulnative_amd import codebook
        lib = _lib.load()
        w = w32 if w32.is_contiguous() else w32.contiguous()
        out_f, in_f = w.shape
        nt = (in_f + tile - 1) // tile
        dev = w.device
        _, mids, order8 = codebook.encode_tables(dev)
        codes = torch.empty(out_f, nt * tile, dtype=torch.uint8, device=dev)
        sc = torch.empty(out_f, nt, dtype=torch.float32, device=dev)
        bad = torch.empty(1, dtype=torch.int64, device=dev)
        with torch.cuda.device(dev):
            rc = lib.smaul_fp8_quantize_tiles(w.data_ptr(), out_f, in_f, tile, order8.data_ptr(), mids.data_ptr(),
                                              codes.data_ptr(), nt * tile, sc.data_ptr(), bad.data_ptr(),
                                              _stream_handle(dev))
        _lib.check(rc, "fp8_quantize_tiles")
        return codes, sc, int(bad.item())

    # ---- linear attention (compute.py:265-322, attn_cpu.cpp) ---------------
    @staticmethod
    def _attn_check(name, eps, tensors):
        _need_device(name, *tensors)
        for t in tensors:
            if t.dtype != torch.float32:
                raise RuntimeError(f"{name}: tensors must be float32, got {t.dtype}")
        if not math.isfinite(eps) or eps <= 0:
            raise RuntimeError(f"{name}: eps must be positive finite, got {eps!r}")

    def attn_forward(self, Q, K, V, eps, need_den, need_state=False):
        """(Y, DEN, S, z) as the reference backend returns them (compute.py:265-289).

        Q/K/V fp32 [B,T,H,D] on the device (K raw, normalised inside).  DEN
        [B,T,H] when ``need_den`` else None.  S [B,H,D,D] / z [B,H,D], the
        final recurrent state, only when ``need_state``; otherwise
        zero-element placeholders, as the native CPU backend returns them.
        Bit-identical to the reference's attn_cpu.cpp on the same inputs.
        """
        lib = _lib.load()
        self._attn_check("attn_forward", eps, (Q, K, V))
        if Q.dim() != 4 or K.shape != Q.shape or V.shape != Q.shape:
            raise RuntimeError("attn_forward: Q/K/V must be [B,T,H,D] with matching shapes")
        B, T, H, D = Q.shape
        if D <= 0 or D > 2048:
            raise RuntimeError(f"attn_forward: D={D} out of the supported range (0, 2048]")
        Qc, Kc, Vc = (t if t.is_contiguous() else t.contiguous() for t in (Q, K, V))
        dev = Q.device
        Y = torch.empty_like(Qc)
        DEN = torch.empty(B, T, H, dtype=torch.float32, device=dev) if need_den else None
        if need_state:
            S = torch.empty(B, H, D, D, dtype=torch.float32, device=dev)
            z = torch.empty(B, H, D, dtype=torch.float32, device=dev)
        else:
            S = torch.empty(0, dtype=torch.float32, device=dev)
            z = torch.empty(0, dtype=torch.float32, device=dev)
        ws_bytes = lib.smaul_attn_workspace_size(B, H, D, int(bool(need_state)))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
        with torch.cuda.device(dev):
            rc = lib.smaul_attn_forward(Qc.data_ptr(), Kc.data_ptr(), Vc.data_ptr(), Y.data_ptr(),
                                        None if DEN is None else DEN.data_ptr(),
                                        S.data_ptr() if need_state else None, z.data_ptr() if need_state else None,
                                        B, T, H, D, float(eps), None if ws is None else ws.data_ptr(), ws_bytes,
                                        _stream_handle(dev))
        _lib.check(rc, "attn_forward")
        return Y, DEN, S, z

    def attn_step(self, S, z, q, k, v, eps):
        """One decode step advancing (S, z) in place; returns (y [B,H,D], S, z)
        (compute.py:291-309, attn_cpu.cpp:421-492, bit-identical)."""
        lib = _lib.load()
        self._attn_check("attn_step", eps, (S, z, q, k, v))
        if q.dim() != 3 or k.shape != q.shape or v.shape != q.shape:
            raise RuntimeError("attn_step: q/k/v must be [B,H,D] with matching shapes")
        B, H, D = q.shape
        if tuple(S.shape) != (B, H, D, D) or tuple(z.shape) != (B, H, D):
            raise RuntimeError("attn_step: S must be [B,H,D,D] and z [B,H,D]")
        if not (S.is_contiguous() and z.is_contiguous()):
            raise RuntimeError("attn_step: the state S and z must be contiguous (they are updated in place)")
        if D <= 0 or D > 2048:
            raise RuntimeError(f"attn_step: D={D} out of the supported range (0, 2048]")
        qc, kc, vc = (t if t.is_contiguous() else t.contiguous() for t in (q, k, v))
        y = torch.empty_like(qc)
        with torch.cuda.device(q.device):
            rc = lib.smaul_attn_step(S.data_ptr(), z.data_ptr(), qc.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                     y.data_ptr(), B, H, D, float(eps), _stream_handle(q.device))
        _lib.check(rc, "attn_step")
        return y, S, z

    def attn_backward(self, dY, Q, K, V, Y, DEN, eps):
        """(dQ, dK, dV) fp32 [B,T,H,D] of the recurrence (compute.py:314-322,
        attn_cpu.cpp:227-368, bit-identical), from the upstream gradient dY and
        the forward's Q, K (raw), V, Y and DEN.  The reference falls back to
        autograd through its torch recurrence when DEN is missing; here the
        forward is run again on the device for it, so the kernel is the same."""
        lib = _lib.load()
        if DEN is None:
            Y, DEN = self.attn_forward(Q, K, V, eps, True)[:2]
        self._attn_check("attn_backward", eps, (dY, Q, K, V, Y, DEN))
        if Q.dim() != 4 or any(t.shape != Q.shape for t in (K, V, dY, Y)):
            raise RuntimeError("attn_backward: Q/K/V/dY/Y must be [B,T,H,D] with matching shapes")
        B, T, H, D = Q.shape
        if tuple(DEN.shape) != (B, T, H):
            raise RuntimeError(f"attn_backward: DEN must be [{B},{T},{H}], got {tuple(DEN.shape)}")
        if D <= 0 or D > 2048:
            raise RuntimeError(f"attn_backward: D={D} out of the supported range (0, 2048]")
        dYc, Qc, Kc, Vc, Yc, DENc = (t if t.is_contiguous() else t.contiguous() for t in (dY, Q, K, V, Y, DEN))
        dev = Q.device
        dQ, dK, dV = torch.empty_like(Qc), torch.empty_like(Qc), torch.empty_like(Qc)
        ws_bytes = lib.smaul_attn_workspace_size(B, H, D, 0)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
        with torch.cuda.device(dev):
            rc = lib.smaul_attn_backward(dYc.data_ptr(), Qc.data_ptr(), Kc.data_ptr(), Vc.data_ptr(), Yc.data_ptr(),
                                         DENc.data_ptr(), dQ.data_ptr(), dK.data_ptr(), dV.data_ptr(), B, T, H, D,
                                         float(eps), None if ws is None else ws.data_ptr(), ws_bytes,
                                         _stream_handle(dev))
        _lib.check(rc, "attn_backward")
        return dQ, dK, dV

    def sparse_grad_v(self, dout, x, cols, values, budget=1 << 22):
        raise NotImplementedError("rocm backend: sparse_grad_v is not implemented")

    # ---- MoE (model.py:557-585) -------------------------------------------
    def _expert_entry(self, experts: Sequence[Sequence[torch.Tensor]], device, d, h, tile):
        """The repack cache entry of a set of experts: ``table``, a device int64
        [6, E] table of the experts' buffer addresses, ``ptrs``, the same
        addresses as host ints, and ``flags``, the C-ABI flags that describe
        the buffers they point at.

        Rows: gate codes, gate scales, up codes, up scales, down codes, down
        scales.  The code rows point at *canonical copies* of the ``w8``
        buffers (0x7F/0xFF rewritten to 0x7E/0xFE, the same +-448 values) so
        the GEMMs can use the hardware E4M3 converter directly; the stored
        ``w8`` buffers are never modified.  With tile 64 and d, h multiples of
        64 the copies are in the tiled layout (``smaul_fp8_tile_layout``:
        each 64-wide K block of consecutive columns contiguous, scales K-major
        in fp32), which the GEMMs stage in whole cache lines; otherwise the
        codes keep FP8Linear's layout, fp32 contiguous scales are used in place
        and other scales (a model cast to bf16) are widened into copies.

        The cache is keyed on the buffers' addresses and holds only weak
        references to them.  When a buffer's ``_version`` changes (requant,
        ``copy_``), the copies are refreshed in place on the current stream,
        so the table -- and any HIP graph that captured it -- keeps pointing
        at valid, current data.  When any of the buffers is freed, its entry
        (and the copies it owns, one byte per weight) is dropped at once; so
        is an entry whose buffers got new storage (a new key for the same
        tensors).  The finalizers hold only weak references to the entry.
        """
        lib = _lib.load()
        flat = []
        for ex in experts:
            if len(ex) != 6:
                raise ValueError("each expert is (gate_w8, gate_sc, up_w8, up_sc, down_w8, down_sc)")
            flat.extend(ex)
        key = (str(device), d, h, tile, tuple(t.data_ptr() for t in flat))
        versions = tuple(t._version for t in flat)
        with self._lock:
            ent = self._ptr_cache.get(key)
        if ent is not None and all(r() is t for r, t in zip(ent["refs"], flat)):
            if ent["versions"] != versions:
                self._refresh(ent, flat, lib, device)
                ent["versions"] = versions
            return ent
        nt_d = (d + tile - 1) // tile
        nt_h = (h + tile - 1) // tile
        shapes = [(h, d), (h, nt_d), (h, d), (h, nt_d), (d, h), (d, nt_h)]
        for n, t in enumerate(flat):
            e, idx = divmod(n, 6)
            if not t.is_cuda or t.device != device:
                raise RuntimeError(f"moe_forward: expert {e} buffer {idx} on {t.device}, x on {device}")
            if tuple(t.shape) != shapes[idx]:
                raise RuntimeError(f"moe_forward: expert {e} buffer {idx} has shape {tuple(t.shape)}, "
                                   f"expected {shapes[idx]}")
            if idx % 2 == 0 and t.dtype != torch.uint8:
                raise RuntimeError(f"moe_forward: expert {e} codes must be uint8, got {t.dtype}")
        tiled = tile == 64 and d % 64 == 0 and h % 64 == 0
        copies = [torch.empty(t.numel(), dtype=torch.uint8, device=device) if i % 2 == 0 else
                  (torch.empty(t.numel(), dtype=torch.float32, device=device) if tiled else None)
                  for i, t in enumerate(flat)]
        flags = _lib.FLAG_CANONICAL_CODES | _lib.FLAG_ALIGNED_CODES | (_lib.FLAG_TILED_LAYOUT if tiled else 0)
        ent = _CacheEntry(copies=copies, refs=[weakref.ref(t) for t in flat], versions=versions, tiled=tiled,
                          flags=flags)
        self._refresh(ent, flat, lib, device)
        E = len(experts)
        rows = [[0] * E for _ in range(6)]
        for n, t in enumerate(flat):
            e, idx = divmod(n, 6)
            src = ent["copies"][n]
            rows[idx][e] = (src if src is not None else t).data_ptr()
        ent["ptrs"] = rows
        ent["table"] = torch.tensor(rows, dtype=torch.int64).to(device)
        ids = {id(t) for t in flat}
        with self._lock:
            # A buffer whose storage was swapped (``sc.data = sc.data.float()``)
            # has a new address, so a new key: drop the entries made for it.
            for k in [k for k, e in self._ptr_cache.items()
                      if any(id(r()) in ids for r in e["refs"] if r() is not None)]:
                del self._ptr_cache[k]
            self._ptr_cache[key] = ent
        me, er = weakref.ref(self), weakref.ref(ent)
        for t in flat:
            weakref.finalize(t, _drop_entry, me, key, er)
        return ent

    def prepare_experts(self, experts, d, h, tile):
        """Build the repack cache entry of a set of expert buffers ahead of the
        first forward (the loader calls this after reading a checkpoint)."""
        if not experts or not experts[0][0].is_cuda:
            raise RuntimeError("prepare_experts: rocm backend needs HIP device tensors")
        self._expert_entry(experts, experts[0][0].device, d, h, tile)

    def _evict(self, key, ent):
        with self._lock:
            if self._ptr_cache.get(key) is ent:
                del self._ptr_cache[key]

    @staticmethod
    def _refresh(ent, flat, lib, device):
        """(Re)write the cached canonical codes and widened scales from the source buffers."""
        stream = _stream_handle(device)
        if ent["tiled"]:
            for n in range(0, len(flat), 2):
                codes, sc = flat[n], flat[n + 1]
                codes = codes if codes.is_contiguous() else codes.contiguous()
                sc = sc if (sc.dtype == torch.float32 and sc.is_contiguous()) else sc.float().contiguous()
                N, K = codes.shape
                with torch.cuda.device(device):
                    rc = lib.smaul_fp8_tile_layout(codes.data_ptr(), sc.data_ptr(), ent["copies"][n].data_ptr(),
                                                   ent["copies"][n + 1].data_ptr(), N, K, stream)
                _lib.check(rc, "fp8_tile_layout")
            return
        for n, t in enumerate(flat):
            if n % 2 == 0:
                src = t if t.is_contiguous() else t.contiguous()
                dst = ent["copies"][n]
                with torch.cuda.device(device):
                    rc = lib.smaul_fp8_canonicalize(src.data_ptr(), dst.data_ptr(), src.numel(), stream)
                _lib.check(rc, "fp8_canonicalize")
            elif not (t.dtype == torch.float32 and t.is_contiguous()):
                w = t.float().contiguous().reshape(-1)
                if ent["copies"][n] is None:
                    ent["copies"][n] = w
                else:
                    ent["copies"][n].copy_(w)

    def swiffn_forward(self, x, buffers, tile):
        """SwiFFN.forward (model.py:289-290) on the device: one fused gate+up
        launch with the SwiGLU epilogue, then the down projection.

        x: [..., d] bf16 or fp32; buffers: (gate_w8, gate_sc, up_w8, up_sc,
        down_w8, down_sc) as FP8Linear stores them.  Returns a new tensor of
        x's dtype and shape, rounded at the points of the reference module
        (each FP8Linear output and the SwiGLU product cast to x.dtype).
        """
        lib = _lib.load()
        _need_device("swiffn_forward", x, *buffers)
        if x.dtype not in _ACT:
            raise RuntimeError(f"swiffn_forward: x must be float32 or bfloat16, got {x.dtype}")
        if tile <= 0:
            raise ValueError(f"tile must be > 0, got {tile}")
        d = x.shape[-1]
        h = buffers[0].shape[0]
        x2 = x.reshape(-1, d)
        x2 = x2 if x2.is_contiguous() else x2.contiguous()
        rows = x2.shape[0]
        dev = x.device
        ent = self._expert_entry([buffers], dev, d, h, tile)
        ptrs = ent["ptrs"]
        out = torch.empty_like(x2)
        ws_bytes = lib.smaul_swiffn_workspace_size(rows, h, _ACT[x.dtype])
        ws = torch.empty(max(1, ws_bytes), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            rc = lib.smaul_swiffn_forward(x2.data_ptr(), _ACT[x.dtype], *[ptrs[i][0] for i in range(6)],
                                          out.data_ptr(), ws.data_ptr(), ws_bytes, rows, d, h, tile,
                                          ent["flags"], _stream_handle(dev))
        _lib.check(rc, "swiffn_forward")
        return out.reshape(x.shape)

    def moe_router(self, x2, gate_w, gate_b, top_k):
        """Router stage alone: (prob [T,E] fp32, topi [T,k] int64, topw [T,k] fp32)."""
        lib = _lib.load()
        _need_device("moe_router", x2, gate_w, gate_b)
        if x2.dtype not in _ACT or x2.dim() != 2:
            raise RuntimeError(f"moe_router: x must be 2-D float32 or bfloat16, got {x2.dtype} {tuple(x2.shape)}")
        T, d = x2.shape
        E = gate_w.shape[0]
        if gate_w.dim() != 2 or gate_w.shape[1] != d:
            raise RuntimeError(f"moe_router: gate weight must be [E, {d}], got {tuple(gate_w.shape)}")
        if gate_b is not None and gate_b.numel() != E:
            raise RuntimeError(f"moe_router: gate bias must have {E} elements, got {gate_b.numel()}")
        x2 = x2 if x2.is_contiguous() else x2.contiguous()
        prob = torch.empty(T, E, dtype=torch.float32, device=x2.device)
        topi = torch.empty(T, top_k, dtype=torch.int64, device=x2.device)
        topw = torch.empty(T, top_k, dtype=torch.float32, device=x2.device)
        gw = gate_w.detach().float().contiguous()
        gb = None if gate_b is None else gate_b.detach().float().contiguous()
        with torch.cuda.device(x2.device):
            rc = lib.smaul_moe_router(x2.data_ptr(), _ACT[x2.dtype], gw.data_ptr(),
                                      None if gb is None else gb.data_ptr(), prob.data_ptr(),
                                      topi.data_ptr(), topw.data_ptr(), T, d, E, top_k,
                                      _stream_handle(x2.device))
        _lib.check(rc, "moe_router")
        return prob, topi, topw

    def moe_dispatch(self, topi, topw, num_experts, block_m=None):
        """Dispatch stage alone: dict of counts/seg_off/tile_off/perm_row/perm_w/inv."""
        lib = _lib.load()
        _need_device("moe_dispatch", topi, topw)
        if topi.dtype != torch.int64 or topw.dtype != torch.float32 or topi.dim() != 2 or \
                tuple(topw.shape) != tuple(topi.shape):
            raise RuntimeError(f"moe_dispatch: topi int64 [T, k] and topw float32 [T, k] expected, got "
                               f"{topi.dtype} {tuple(topi.shape)} / {topw.dtype} {tuple(topw.shape)}")
        T, k = topi.shape
        E = int(num_experts)
        if block_m is None:
            block_m = 32
        dev = topi.device
        i32 = dict(dtype=torch.int32, device=dev)
        out = {
            "counts": torch.empty(E, **i32),
            "seg_off": torch.empty(E + 1, **i32),
            "tile_off": torch.empty(E + 1, **i32),
            "perm_row": torch.empty(max(1, T * k), **i32),
            "perm_w": torch.empty(max(1, T * k), dtype=torch.float32, device=dev),
            "inv": torch.empty(max(1, T * k), **i32),
        }
        ws_bytes = lib.smaul_moe_dispatch_workspace_size(T, E)
        ws = torch.empty(max(1, ws_bytes), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            rc = lib.smaul_moe_dispatch(topi.contiguous().data_ptr(), topw.contiguous().data_ptr(),
                                        out["counts"].data_ptr(), out["seg_off"].data_ptr(),
                                        out["tile_off"].data_ptr(), out["perm_row"].data_ptr(),
                                        out["perm_w"].data_ptr(), out["inv"].data_ptr(), T, E, k,
                                        block_m, ws.data_ptr(), ws_bytes, _stream_handle(dev))
        _lib.check(rc, "moe_dispatch")
        out["block_m"] = block_m
        return out

    def moe_stages(self, x2, gate_w, gate_b, experts, top_k, tile, events=None, block_m=None):
        """The MoE layer as its five stages, each through its own C-ABI entry.

        Same results as ``moe_forward`` (which runs the same kernels from one
        call).  ``events``, if given, is a list of 6 ``torch.cuda.Event``
        recorded on the current stream before the router and after each stage
        (router, dispatch, gate_up, down, combine), for per-kernel timing.
        ``block_m`` overrides ``smaul_moe_block_m``'s tile height (64: the
        64-row LDS-DMA tiles that ``moe_forward`` takes for small layers).
        Returns (out [T,d], prob, topi, topw, dispatch dict).
        """
        lib = _lib.load()
        _need_device("moe_stages", x2, gate_w, gate_b)
        if x2.dtype not in _ACT or x2.dim() != 2:
            raise RuntimeError(f"moe_stages: x must be 2-D float32 or bfloat16, got {x2.dtype} {tuple(x2.shape)}")
        x2 = x2 if x2.is_contiguous() else x2.contiguous()
        T, d = x2.shape
        E = len(experts)
        h = experts[0][0].shape[0]
        dev = x2.device
        act = _ACT[x2.dtype]
        ent = self._expert_entry(experts, dev, d, h, tile)
        table, eflags = ent["table"], ent["flags"]
        gw = gate_w.detach().float().contiguous()
        gb = None if gate_b is None else gate_b.detach().float().contiguous()
        R = T * top_k
        bm = lib.smaul_moe_block_m(T, d, h, E, top_k, tile, act) if block_m is None else int(block_m)
        max_tiles = (R + bm - 1) // bm + E
        hdn = torch.empty(max(1, R), h, dtype=x2.dtype, device=dev)
        yperm = torch.empty(max(1, R), d, dtype=x2.dtype, device=dev)
        out = torch.empty_like(x2)
        stream = torch.cuda.current_stream(dev)
        rec = (lambda i: events[i].record(stream)) if events else (lambda i: None)
        tp = table.data_ptr()
        row = E * 8
        with torch.cuda.device(dev):
            rec(0)
            prob, topi, topw = self.moe_router(x2, gw, gb, top_k)
            rec(1)
            disp = self.moe_dispatch(topi, topw, E, bm)
            rec(2)
            sh = stream.cuda_stream
            rc = lib.smaul_moe_gate_up(x2.data_ptr(), act, disp["perm_row"].data_ptr(), tp, tp + row,
                                       tp + 2 * row, tp + 3 * row, hdn.data_ptr(), disp["seg_off"].data_ptr(),
                                       disp["tile_off"].data_ptr(), max_tiles, E, d, h, tile, bm, eflags, sh)
            _lib.check(rc, "moe_gate_up")
            rec(3)
            rc = lib.smaul_moe_down(hdn.data_ptr(), act, tp + 4 * row, tp + 5 * row, yperm.data_ptr(),
                                    disp["seg_off"].data_ptr(), disp["tile_off"].data_ptr(), max_tiles, E, d,
                                    h, tile, bm, eflags, sh)
            _lib.check(rc, "moe_down")
            rec(4)
            rc = lib.smaul_moe_combine(yperm.data_ptr(), act, topi.data_ptr(), topw.data_ptr(),
                                       disp["inv"].data_ptr(), out.data_ptr(), T, d, top_k, sh)
            _lib.check(rc, "moe_combine")
            rec(5)
        disp["hdn"] = hdn
        disp["yperm"] = yperm
        return out, prob, topi, topw, disp

    def rms_norm(self, x, weight=None, eps=1e-6):
        """RMSNorm.forward (model.py:124-139) over the last dim, on the device.

        x: [..., d] bf16 or fp32; weight: [d] (None = ones, the unit-RMS norm).
        Returns a new tensor of x's dtype and shape.
        """
        lib = _lib.load()
        _need_device("rms_norm", x, weight)
        if x.dtype not in _ACT:
            raise RuntimeError(f"rms_norm: x must be float32 or bfloat16, got {x.dtype}")
        if not math.isfinite(eps) or eps <= 0:
            raise ValueError(f"RMSNorm eps must be positive finite, got {eps!r}")
        d = x.shape[-1]
        x2 = x.reshape(-1, d)
        x2 = x2 if x2.is_contiguous() else x2.contiguous()
        w = None
        if weight is not None:
            if weight.numel() != d:
                raise RuntimeError(f"rms_norm: weight must have {d} elements, got {weight.numel()}")
            w = weight.detach().reshape(d)
            w = w if (w.dtype == torch.float32 and w.is_contiguous()) else w.float().contiguous()
        out = torch.empty_like(x2)
        with torch.cuda.device(x.device):
            rc = lib.smaul_rms_norm(x2.data_ptr(), _ACT[x.dtype], None if w is None else w.data_ptr(),
                                    out.data_ptr(), x2.shape[0], d, eps, _stream_handle(x.device))
        _lib.check(rc, "rms_norm")
        return out.reshape(x.shape)

    def wait_timeouts(self, device=None, reset=False) -> int:
        """Give-ups of the decode combine's bounded wait on ``device`` since the
        library was loaded or last reset (``reset=True`` clears what it reads).

        In the decode regime the combine runs in the tail of the down kernel,
        whose first workgroups wait for the others.  A wait that gives up
        writes NaN over the tokens it owns (and -1 over their next top-k ids)
        instead of combining rows that may not have been written, and counts
        itself here.  The count is read back to the host, so this call waits
        for the work already queued on the current stream."""
        lib = _lib.load()
        dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        buf = torch.empty(1, dtype=torch.int32, device=dev)
        with torch.cuda.device(dev):
            rc = lib.smaul_wait_timeouts(buf.data_ptr(), int(bool(reset)), _stream_handle(dev))
        _lib.check(rc, "wait_timeouts")
        return int(buf.item())

    def moe_forward(self, x, gate_w, gate_b, experts, top_k, tile):
        """SwiFFN_MoE.forward on the device.

        x: [..., d] bf16 or fp32; gate_w fp32 [E, d]; gate_b [E] or None;
        experts: E tuples (gate_w8, gate_sc, up_w8, up_sc, down_w8, down_sc).
        Returns (out [..., d] x.dtype, prob [..., E] fp32, topi [..., k] int64,
        counts [E] int32 on the device).
        """
        return self._moe_forward(x, gate_w, gate_b, experts, top_k, tile, None)

    def moe_forward_norm(self, x, gate_w, gate_b, experts, top_k, tile, norm_weight=None, eps=1e-6,
                         routing=None, next_router=None):
        """moe_forward followed by RMSNorm of its output (Block's norm of the
        FFN output, model.py:636), fused into the combine where the shape
        allows.  Returns moe_forward's tuple plus the normalised output, which
        equals rms_norm(out, norm_weight, eps) bit for bit.

        For a chain of layers (each layer's normalised output is the next
        layer's input, model.py:636 into the next router, model.py:558-570):
        - routing=(prob, topi, topw): this layer's routing of x, computed
          before (moe_router's outputs, or the previous call's next routing);
          the layer runs no router and returns prob/topi as given.
        - next_router=(gate_w, gate_b, top_k): the next layer's router; the
          normalised output is routed with it (inside the combine kernel
          where the shape allows) and (prob, topi, topw) is appended to the
          returned tuple, equal bit for bit to moe_router(normed, ...)."""
        if not math.isfinite(eps) or eps <= 0:
            raise ValueError(f"RMSNorm eps must be positive finite, got {eps!r}")
        return self._moe_forward(x, gate_w, gate_b, experts, top_k, tile, (norm_weight, eps), routing,
                                 next_router)

    def _moe_forward(self, x, gate_w, gate_b, experts, top_k, tile, norm, routing=None, next_router=None):
        lib = _lib.load()
        _need_device("moe_forward", x, gate_w, gate_b, None if norm is None else norm[0])
        if x.dtype not in _ACT:
            raise RuntimeError(f"moe_forward: x must be float32 or bfloat16, got {x.dtype}")
        d = x.shape[-1]
        E = len(experts)
        if gate_w.dim() != 2 or tuple(gate_w.shape) != (E, d):
            raise RuntimeError(f"moe_forward: gate weight must be [{E}, {d}], got {tuple(gate_w.shape)}")
        if gate_b is not None and gate_b.numel() != E:
            raise RuntimeError(f"moe_forward: gate bias must have {E} elements, got {gate_b.numel()}")
        if not 1 <= top_k <= E:
            raise ValueError(f"top_k must be in [1, {E}], got {top_k}")
        if tile <= 0:
            raise ValueError(f"tile must be > 0, got {tile}")
        h = experts[0][0].shape[0]
        x2 = x.reshape(-1, d)
        x2 = x2 if x2.is_contiguous() else x2.contiguous()
        T = x2.shape[0]
        dev = x.device
        ent = self._expert_entry(experts, dev, d, h, tile)
        table, eflags = ent["table"], ent["flags"]
        gw = gate_w.detach()
        gw = gw if (gw.dtype == torch.float32 and gw.is_contiguous()) else gw.float().contiguous()
        gb = None
        if gate_b is not None:
            gb = gate_b.detach()
            gb = gb if (gb.dtype == torch.float32 and gb.is_contiguous()) else gb.float().contiguous()
        act = _ACT[x.dtype]
        out = torch.empty_like(x2)
        if routing is None:
            prob = torch.empty(T, E, dtype=torch.float32, device=dev)
            topi = torch.empty(T, top_k, dtype=torch.int64, device=dev)
            topw = torch.empty(T, top_k, dtype=torch.float32, device=dev)
        else:
            prob, topi, topw = routing
            _need_device("moe_forward", x, prob, topi, topw)
            for name, t, dt, shape in (("prob", prob, torch.float32, (T, E)), ("topi", topi, torch.int64, (T, top_k)),
                                       ("topw", topw, torch.float32, (T, top_k))):
                if t.dtype != dt or tuple(t.shape) != shape or not t.is_contiguous():
                    raise RuntimeError(f"moe_forward: routing {name} must be contiguous {dt} {list(shape)}, "
                                       f"got {t.dtype} {list(t.shape)}")
        nxt = None
        if next_router is not None:
            ngw, ngb, nk = next_router
            _need_device("moe_forward", x, ngw, ngb)
            nE = ngw.shape[0]
            if ngw.dim() != 2 or ngw.shape[1] != d:
                raise RuntimeError(f"moe_forward: next gate weight must be [E, {d}], got {tuple(ngw.shape)}")
            if not 1 <= nk <= nE:
                raise ValueError(f"next top_k must be in [1, {nE}], got {nk}")
            ngw = ngw.detach()
            ngw = ngw if (ngw.dtype == torch.float32 and ngw.is_contiguous()) else ngw.float().contiguous()
            if ngb is not None:
                ngb = ngb.detach()
                ngb = ngb if (ngb.dtype == torch.float32 and ngb.is_contiguous()) else ngb.float().contiguous()
            nxt = (ngw, ngb, nE, nk, torch.empty(T, nE, dtype=torch.float32, device=dev),
                   torch.empty(T, nk, dtype=torch.int64, device=dev), torch.empty(T, nk, dtype=torch.float32, device=dev))
        # the dispatch kernel writes every count; no fill, so the call can be graph-captured
        counts = torch.empty(E, dtype=torch.int32, device=dev) if T > 0 else \
            torch.zeros(E, dtype=torch.int32, device=dev)
        normed = nw = None
        if norm is not None:
            normed = torch.empty_like(x2)
            if norm[0] is not None:
                if norm[0].numel() != d:
                    raise RuntimeError(f"moe_forward_norm: weight must have {d} elements, got {norm[0].numel()}")
                nw = norm[0].detach().reshape(d)
                nw = nw if (nw.dtype == torch.float32 and nw.is_contiguous()) else nw.float().contiguous()
        if T > 0:
            ws_bytes = lib.smaul_moe_workspace_size(T, d, h, E, top_k, act)
            if ws_bytes < 0:
                raise ValueError("moe_forward: invalid sizes")
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
            tp = table.data_ptr()
            row = E * 8
            args = [x2.data_ptr(), act, gw.data_ptr(), None if gb is None else gb.data_ptr(),
                    tp, tp + row, tp + 2 * row, tp + 3 * row, tp + 4 * row, tp + 5 * row,
                    out.data_ptr(), prob.data_ptr(), topi.data_ptr(), topw.data_ptr(),
                    counts.data_ptr(), ws.data_ptr(), ws_bytes, T, d, h, E, top_k, tile, eflags]
            with torch.cuda.device(dev):
                if norm is None:
                    rc = lib.smaul_moe_forward(*args, _stream_handle(dev))
                elif routing is None and nxt is None:
                    rc = lib.smaul_moe_forward_norm(*args, None if nw is None else nw.data_ptr(), norm[1],
                                                    normed.data_ptr(), _stream_handle(dev))
                else:
                    nargs = [None] * 7 if nxt is None else \
                        [nxt[0].data_ptr(), None if nxt[1] is None else nxt[1].data_ptr(), nxt[2], nxt[3],
                         nxt[4].data_ptr(), nxt[5].data_ptr(), nxt[6].data_ptr()]
                    if nxt is None:
                        nargs[2] = nargs[3] = 0
                    rc = lib.smaul_moe_forward_chain(*args, None if nw is None else nw.data_ptr(), norm[1],
                                                     normed.data_ptr(), int(routing is not None), *nargs,
                                                     _stream_handle(dev))
            _lib.check(rc, "moe_forward")
        lead = x.shape[:-1]
        res = (out.reshape(*lead, d), prob.reshape(*lead, E), topi.reshape(*lead, top_k), counts)
        if norm is None:
            return res
        res = res + (normed.reshape(*lead, d),)
        if nxt is not None:
            res = res + ((nxt[4].reshape(*lead, nxt[2]), nxt[5].reshape(*lead, nxt[3]),
                          nxt[6].reshape(*lead, nxt[3])),)
        return res
