"""CPU oracle for the tiled-FP8 MoE forward path.

TEST INFRASTRUCTURE ONLY.  This package restates the reference algorithm on
the CPU so the HIP kernels can be checked against it.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import it,
and only as the checker: the product (``smaulnative_amd``) never imports,
links or calls anything here.

Pieces and the reference code each one follows (paths under the reference
checkout):

- ``e4m3_lut``          kernel/fp8_tile.py:39-48, kernel/fp8_cpu.cpp:16-26
- ``quant_tables``      kernel/fp8_tile.py:49-53 (torch.argsort order + midpoints)
- ``quantize_tiles``    kernel/fp8_tile.py:82-119 (the torch path)
- ``decode_tile``       kernel/fp8_tile.py:121-131
- ``fp8_forward``       kernel/fp8_cpu.cpp:49-141 via ``fp8_gemm.c`` (C, bit-exact)
- ``fp8_backward_input`` kernel/fp8_cpu.cpp:167-259 via ``fp8_gemm.c`` (C, bit-exact)
- ``fp8_linear``        kernel/fp8_tile.py:163-170 (_Fn.forward dtype handling)
- ``swiffn_forward``    model.py:289-290
- ``moe_forward``       model.py:557-585 (router, top-k, mask dispatch, combine)
- ``attn_forward``      kernel/attn_cpu.cpp:16-24,40-142 via ``attn.c`` (C, bit-exact)
- ``attn_step``         kernel/attn_cpu.cpp:421-492 via ``attn.c``
- ``attn_textbook``     model.py:199-218 (_attn_reference: the same recurrence in torch ops)

Arithmetic that lives in torch (router GEMM, softmax, topk, silu) is computed
with the same torch CPU calls the reference makes; torch is a third-party
dependency pinned by the reference only as ``torch>=2.0,<3.0``
(requirements.txt:1).

How each piece is pinned (tests/test_oracle.py):
- LUT: closed form of E4M3 with the +-448 convention, and the reference's
  golden table (tests/golden/).
- fp8_forward: bit-exact against the reference's own fp8_cpu.cpp built under
  oracle/_ref (when present), against golden vectors written from it, and
  against brute force x @ decode(W).T on tiny shapes.
- fp8_backward_input: bit-exact against the same reference build on shapes
  that take both of its arithmetic orders, and against g @ decode(W).
- quantize_tiles: golden codes/scales from the reference quantizer on the
  special-value cases of tests/test_linear_fp8.py:484-510.
- moe_forward: golden outputs, probabilities, top-k indices and counts of the
  reference SwiFFN_MoE, including exact-tie and zero-weight routing cases.
- attn_forward / attn_step: bit-exact against the reference's own attn_cpu.cpp
  built under oracle/_ref and against golden vectors written from it; within
  fp32 rounding of the textbook recurrence (model.py:199-218); closed forms at
  T=1 (y = v when q.kn >= eps) and for zero keys (the 1e-6 clamp).
"""
from __future__ import annotations

import ctypes
import glob
import importlib.util
import os
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np
import torch
import torch.nn.functional as F

TILE = 64
E4M3_MAX = 448.0
_HERE = os.path.dirname(os.path.abspath(__file__))


# --------------------------------------------------------------------------
# codebook
# --------------------------------------------------------------------------
def e4m3_lut() -> np.ndarray:
    """256 fp32 values of the reference E4M3 codebook (fp8_tile.py:39-48).

    e=(c>>3)&15, m=c&7; e=15,m=7 -> +-448 (not NaN as in OCP E4M3FN);
    e=0 -> +-m*2^-9; otherwise +-(1+m/8)*2^(e-7).
    """
    v = np.empty(256, dtype=np.float32)
    for c in range(256):
        e, m = (c >> 3) & 15, c & 7
        s = -1.0 if c & 128 else 1.0
        if e == 15 and m == 7:
            v[c] = s * 448.0
        elif e == 0:
            v[c] = s * m * 2.0 ** -9
        else:
            v[c] = s * (1 + m / 8.0) * 2.0 ** (e - 7)
    return v


def quant_tables():
    """(lut, order int64[256], sorted values, midpoints[255]) as fp8_tile.py:49-53.

    ``order`` comes from torch.argsort, the reference's own call, because the
    codebook has duplicate values (0x7E/0x7F = 448, 0xFE/0xFF = -448,
    0x00/0x80 = 0) and the tie order is torch's.
    """
    v = torch.from_numpy(e4m3_lut())
    order = torch.argsort(v)
    sval = v[order]
    bounds = (sval[:-1] + sval[1:]) * 0.5
    return v, order, sval, bounds


def quantize_tiles(w32: torch.Tensor, tile: int = TILE):
    """Tiled E4M3 quantizer, the torch path of fp8_tile.py:82-119.

    Returns (codes uint8 [out_f, in_f], scales fp32 [out_f, ceil(in_f/tile)]).
    """
    if tile <= 0:
        raise ValueError(f"tile must be > 0, got {tile}")
    if w32.dim() != 2:
        raise ValueError("w32 must be 2D")
    out_f, in_f = w32.shape
    w32 = w32.detach().float().contiguous().cpu()
    nt = (in_f + tile - 1) // tile
    pad = nt * tile - in_f
    if pad:
        w32 = torch.cat([w32, torch.zeros(out_f, pad, dtype=w32.dtype)], 1)
    _, order, _, bounds = quant_tables()
    blk = w32.reshape(out_f, nt, tile)
    amax = torch.where(torch.isfinite(blk), blk.abs(), 0.0).amax(dim=2).clamp_min(1e-12)
    sc = (amax / E4M3_MAX).clamp_min(1e-12)
    n = torch.nan_to_num(blk / sc[..., None], nan=0.0).clamp(-E4M3_MAX, E4M3_MAX)
    nf = n.reshape(-1)
    codes = order[torch.bucketize(nf, bounds).clamp(0, 255)].reshape(out_f, nt * tile)
    codes.reshape(-1)[nf == 0] = 0
    return codes[:, :in_f].contiguous().to(torch.uint8), sc


def decode_tile(w, s, o0, o1, t, tile=TILE):
    """fp8_tile.py:121-131: rows [o0:o1] of tile t, decoded to fp32."""
    lut = torch.from_numpy(e4m3_lut())
    blk = w[o0:o1, t * tile:(t + 1) * tile].long()
    return lut[blk] * s[o0:o1, t].float()[:, None]


def decode_full(w, s, tile=TILE):
    """Whole [out_f, in_f] decoded weight, tile by tile (brute-force check)."""
    out_f, in_f = w.shape
    nt = (in_f + tile - 1) // tile
    return torch.cat([decode_tile(w, s, 0, out_f, t, tile)[:, :min(tile, in_f - t * tile)]
                      for t in range(nt)], 1)


# --------------------------------------------------------------------------
# fp8 GEMM (C restatement, or the reference's own kernel from oracle/_ref)
# --------------------------------------------------------------------------
_lib = None
_ref_mod = None


def _load_lib():
    global _lib
    if _lib is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run make -C oracle)")
        lib = ctypes.CDLL(path)
        lib.oracle_fp8_forward.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 4 + [ctypes.c_int]
        lib.oracle_fp8_forward.restype = ctypes.c_int
        lib.oracle_e4m3_lut.argtypes = [ctypes.c_void_p]
        lib.oracle_fp8_backward_input.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 4 + [ctypes.c_int]
        lib.oracle_fp8_backward_input.restype = ctypes.c_int
        lib.oracle_attn_forward.argtypes = [ctypes.c_void_p] * 7 + [ctypes.c_int64] * 4 + [ctypes.c_float]
        lib.oracle_attn_forward.restype = ctypes.c_int
        lib.oracle_attn_step.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int64] * 3 + [ctypes.c_float]
        lib.oracle_attn_step.restype = ctypes.c_int
        lib.oracle_attn_backward.argtypes = [ctypes.c_void_p] * 9 + [ctypes.c_int64] * 4 + [ctypes.c_float]
        lib.oracle_attn_backward.restype = ctypes.c_int
        _lib = lib
    return _lib


def default_threads() -> int:
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:  # pragma: no cover
        return max(1, os.cpu_count() or 1)


def c_lut() -> np.ndarray:
    out = np.empty(256, dtype=np.float32)
    _load_lib().oracle_e4m3_lut(out.ctypes.data)
    return out


def fp8_forward(x, w, s, in_f, out_f, tile=TILE, threads: Optional[int] = None):
    """Reference fp8_forward semantics (fp8_cpu.cpp:100-141), C restatement.

    x fp32 [rows, in_f]; w uint8 [out_f, in_f] (or flat); s fp32 [out_f, nt]
    (or flat).  Returns fp32 [rows, out_f].
    """
    if tile <= 0 or in_f <= 0 or out_f <= 0:
        raise ValueError(f"tile/in_f/out_f must be positive, got {tile}/{in_f}/{out_f}")
    xc = x.detach().cpu().float().contiguous()
    wc = w.detach().cpu().reshape(-1).contiguous()
    sc = s.detach().cpu().float().reshape(-1).contiguous()
    rows = xc.shape[0]
    nt = (in_f + tile - 1) // tile
    assert xc.shape[1] == in_f and wc.numel() == out_f * in_f and sc.numel() == out_f * nt
    y = torch.empty(rows, out_f, dtype=torch.float32)
    rc = _load_lib().oracle_fp8_forward(xc.data_ptr(), wc.data_ptr(), sc.data_ptr(), y.data_ptr(),
                                        rows, in_f, out_f, tile, threads or default_threads())
    if rc != 0:
        raise RuntimeError(f"oracle_fp8_forward failed ({rc})")
    return y


def fp8_backward_input(g, w, s, in_f, out_f, tile=TILE, threads: Optional[int] = None):
    """Reference fp8_backward_input semantics (fp8_cpu.cpp:167-259), C restatement.

    g fp32 [rows, out_f]; w uint8 [out_f, in_f]; s fp32 [out_f, nt].  Returns
    dx fp32 [rows, in_f] = g . decode(w, s).
    """
    gc = g.detach().cpu().float().contiguous()
    wc = w.detach().cpu().reshape(-1).contiguous()
    sc = s.detach().cpu().float().reshape(-1).contiguous()
    rows = gc.shape[0]
    dx = torch.empty(rows, in_f, dtype=torch.float32)
    rc = _load_lib().oracle_fp8_backward_input(gc.data_ptr(), wc.data_ptr(), sc.data_ptr(), dx.data_ptr(),
                                               rows, in_f, out_f, tile, threads or default_threads())
    if rc != 0:
        raise RuntimeError(f"oracle_fp8_backward_input failed ({rc})")
    return dx


def ref_module():
    """The reference's own fp8_cpu.cpp built by oracle/Makefile, or None."""
    global _ref_mod
    if _ref_mod is None:
        hits = sorted(glob.glob(os.path.join(_HERE, "_ref", "smaul_fp8_ref*.so")))
        if not hits:
            return None
        torch.ops.load_library  # make sure torch's shared libs are loaded first
        spec = importlib.util.spec_from_file_location("smaul_fp8_ref", hits[0])
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _ref_mod = mod
    return _ref_mod


def fp8_forward_ref(x, w, s, in_f, out_f, tile=TILE):
    """The reference kernel itself (oracle/_ref); raises if it is not built."""
    mod = ref_module()
    if mod is None:
        raise RuntimeError("oracle/_ref not built")
    return mod.fp8_forward(x.detach().cpu().float().contiguous(), w.cpu().reshape(-1).contiguous(),
                           s.cpu().float().reshape(-1).contiguous(), in_f, out_f, tile)


# --------------------------------------------------------------------------
# modules: FP8Linear forward, SwiFFN, SwiFFN_MoE
# --------------------------------------------------------------------------
def fp8_linear(x, w, s, tile=TILE, gemm=None):
    """_Fn.forward (fp8_tile.py:163-170): fp32 GEMM, result cast to x.dtype."""
    gemm = gemm or fp8_forward
    out_f, in_f = w.shape
    x2 = x.reshape(-1, in_f).float().contiguous()
    y = gemm(x2, w, s, in_f, out_f, tile)
    return y.reshape(*x.shape[:-1], out_f).to(x.dtype)


@dataclass
class ExpertWeights:
    """One SwiFFN expert (model.py:282-288): gate/up [h,d], down [d,h] as codes+scales."""
    gate_w: torch.Tensor
    gate_s: torch.Tensor
    up_w: torch.Tensor
    up_s: torch.Tensor
    down_w: torch.Tensor
    down_s: torch.Tensor


def swiffn_forward(x, ex: ExpertWeights, tile=TILE, gemm=None):
    """model.py:289-290: down((silu(gate(x).float()) * up(x).float()).to(x.dtype))."""
    odt = x.dtype if x.is_floating_point() else torch.float32
    g = fp8_linear(x, ex.gate_w, ex.gate_s, tile, gemm)
    u = fp8_linear(x, ex.up_w, ex.up_s, tile, gemm)
    hdn = (F.silu(g.float()) * u.float()).to(odt)
    return fp8_linear(hdn, ex.down_w, ex.down_s, tile, gemm)


@dataclass
class MoEResult:
    out: torch.Tensor
    prob: torch.Tensor
    topi: torch.Tensor
    topw: torch.Tensor               # renormalised routing weights [.., k]
    counts: List[int]
    executed: List[bool]
    perm: List[torch.Tensor] = field(default_factory=list)   # per expert: token indices


def route(x, gate_w, gate_b, top_k):
    """Router of model.py:558-570: fp32 logits, softmax, topk, renormalise."""
    logits = F.linear(x.float(), gate_w.float(), None if gate_b is None else gate_b.float())
    prob = torch.softmax(logits, -1)
    topv, topi = torch.topk(prob, top_k, -1)
    denom = topv.sum(-1, keepdim=True)
    tiny = denom.squeeze(-1) < 1e-6
    topv = torch.where(tiny.unsqueeze(-1), torch.full_like(topv, 1.0 / top_k),
                       topv / denom.clamp_min(1e-9))
    return prob, topi, topv


def moe_forward(x, gate_w, gate_b, experts: List[ExpertWeights], top_k, tile=TILE, gemm=None,
                expert_fn=None):
    """SwiFFN_MoE.forward (model.py:557-585) on the CPU.

    ``expert_fn(e, xm)`` overrides the expert call (default: ``swiffn_forward``
    with the oracle GEMM).  The per-expert token order (``perm``) is the order
    of the boolean gather x[m]: ascending flattened token index.
    """
    x = x.detach().cpu()
    prob, topi, topv = route(x, gate_w, gate_b, top_k)
    out = torch.zeros_like(x.float())
    E = len(experts)
    counts, executed, perm = [0] * E, [False] * E, []
    flat_m_idx = torch.arange(x.numel() // x.shape[-1]).reshape(x.shape[:-1])
    for e in range(E):
        w = torch.where(topi == e, topv, torch.zeros_like(topv)).sum(-1, keepdim=True)
        m = (w.squeeze(-1) > 0)
        n = int(m.sum().item()) if m.numel() else 0
        counts[e] = n
        perm.append(flat_m_idx[m])
        if m.any():
            executed[e] = True
            xm = x[m].contiguous()
            y = expert_fn(e, xm) if expert_fn else swiffn_forward(xm, experts[e], tile, gemm)
            out[m] += y.float() * w[m]
    res = out.to(x.dtype if x.is_floating_point() else torch.float32)
    return MoEResult(res, prob, topi, topv, counts, executed, perm)


# --------------------------------------------------------------------------
# linear attention (C restatement, the reference's own kernel, textbook form)
# --------------------------------------------------------------------------
def attn_forward(Q, K, V, eps=1e-6):
    """attn_cpu.cpp attn_forward with DEN and the final state: (Y, DEN, S, z).

    Q/K/V fp32 [B,T,H,D] (K raw, post-elu+1; normalised inside).  DEN [B,T,H],
    S [B,H,D,D], z [B,H,D].
    """
    Qc, Kc, Vc = (t.detach().cpu().float().contiguous() for t in (Q, K, V))
    B, T, H, D = Qc.shape
    Y = torch.empty_like(Qc)
    DEN = torch.empty(B, T, H)
    S = torch.empty(B, H, D, D)
    z = torch.empty(B, H, D)
    rc = _load_lib().oracle_attn_forward(Qc.data_ptr(), Kc.data_ptr(), Vc.data_ptr(), Y.data_ptr(),
                                         DEN.data_ptr(), S.data_ptr(), z.data_ptr(), B, T, H, D, eps)
    if rc != 0:
        raise RuntimeError(f"oracle_attn_forward failed ({rc})")
    return Y, DEN, S, z


def attn_step(S, z, q, k, v, eps=1e-6):
    """attn_cpu.cpp attn_step on copies: returns (y [B,H,D], S', z')."""
    S2 = S.detach().cpu().float().contiguous().clone()
    z2 = z.detach().cpu().float().contiguous().clone()
    qc, kc, vc = (t.detach().cpu().float().contiguous() for t in (q, k, v))
    B, H, D = qc.shape
    y = torch.empty_like(qc)
    rc = _load_lib().oracle_attn_step(S2.data_ptr(), z2.data_ptr(), qc.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                      y.data_ptr(), B, H, D, eps)
    if rc != 0:
        raise RuntimeError(f"oracle_attn_step failed ({rc})")
    return y, S2, z2


_ref_attn_mod = None


def attn_backward(dY, Q, K, V, Y, DEN, eps=1e-6):
    """attn_cpu.cpp attn_backward (:227-368): (dQ, dK, dV) fp32 [B,T,H,D] from
    the upstream gradient dY, the forward's inputs (K raw) and its Y, DEN."""
    dYc, Qc, Kc, Vc, Yc, DENc = (t.detach().cpu().float().contiguous() for t in (dY, Q, K, V, Y, DEN))
    B, T, H, D = Qc.shape
    dQ, dK, dV = torch.empty_like(Qc), torch.empty_like(Qc), torch.empty_like(Qc)
    rc = _load_lib().oracle_attn_backward(dYc.data_ptr(), Qc.data_ptr(), Kc.data_ptr(), Vc.data_ptr(), Yc.data_ptr(),
                                          DENc.data_ptr(), dQ.data_ptr(), dK.data_ptr(), dV.data_ptr(), B, T, H, D,
                                          eps)
    if rc != 0:
        raise RuntimeError(f"oracle_attn_backward failed ({rc})")
    return dQ, dK, dV


def ref_attn_module():
    """The reference's own attn_cpu.cpp built by oracle/Makefile, or None."""
    global _ref_attn_mod
    if _ref_attn_mod is None:
        hits = sorted(glob.glob(os.path.join(_HERE, "_ref", "smaul_attn_ref*.so")))
        if not hits:
            return None
        spec = importlib.util.spec_from_file_location("smaul_attn_ref", hits[0])
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _ref_attn_mod = mod
    return _ref_attn_mod


def attn_textbook(Q, K, V, eps=1e-6):
    """model.py:199-218 (_attn_reference): the recurrence in torch ops, fp32."""
    B, T, H, D = Q.shape
    S = torch.zeros(B, H, D, D)
    z = torch.zeros(B, H, D)
    ys = []
    for t in range(T):
        kt, vt, qt = K[:, t].float(), V[:, t].float(), Q[:, t].float()
        kt = kt / kt.norm(dim=-1, keepdim=True).clamp_min(1e-6)
        S = S + kt.unsqueeze(-1) @ vt.unsqueeze(-2)
        z = z + kt
        num = (qt.unsqueeze(-2) @ S).squeeze(-2)
        den = (qt * z).sum(-1, keepdim=True).clamp_min(eps)
        ys.append(num / den)
    return torch.stack(ys, 1) if ys else torch.empty(B, 0, H, D)


# --------------------------------------------------------------------------
# synthetic workloads (seeded; identical host tensors feed CPU and GPU)
# --------------------------------------------------------------------------
def make_expert(d, h, gen, tile=TILE, std=0.02):
    def q(o, i):
        w = torch.randn(o, i, generator=gen) * std
        return quantize_tiles(w, tile)
    gw, gs = q(h, d)
    uw, us = q(h, d)
    dw, ds = q(d, h)
    return ExpertWeights(gw, gs, uw, us, dw, ds)


__all__ = [n for n in dir() if not n.startswith("_")]
