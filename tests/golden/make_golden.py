"""Writes the golden fixtures under tests/golden/ from the reference itself.

Run in the build container only (the reference is not present on the GPU box):

    python tests/golden/make_golden.py

What it pins, and why an import is needed for it: the parts of the path whose
bits live in torch and that no closed form or brute force fixes --
torch.argsort's order between the duplicate codebook values
(kernel/fp8_tile.py:49), torch.topk's order between equal router
probabilities (model.py:564), the fp32 router/softmax bits (model.py:558) and
the dtype rounding points of SwiFFN_MoE.forward (model.py:557-585,289-290).

The reference's fp8 GEMM is its own kernel/fp8_cpu.cpp compiled by
oracle/Makefile into oracle/_ref (its JIT loader is never run); the quantizer
runs the reference's torch path (kernel/fp8_tile.py:100-113), which its tests
hold bit-identical to its native quantizer (tests/test_linear_fp8.py:513-523).
Output: golden_*.npz (inputs and expected outputs, nothing else).
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REF = os.environ.get("SMAUL_REFERENCE", "/root/reference")
sys.path.insert(0, REPO)
sys.path.insert(0, REF)

import oracle  # noqa: E402  (only for oracle/_ref, the reference kernel build)
from kernel import compute as ref_compute  # noqa: E402
from kernel import fp8_tile as ref_fp8  # noqa: E402
import model as ref_model  # noqa: E402


def _backend():
    be = ref_compute.get_backend("cpu")
    mod = oracle.ref_module()
    if mod is None:
        raise SystemExit("build oracle/_ref first: make -C oracle")
    be._ext = mod          # the reference's own fp8_cpu.cpp, built from source here
    be._quant = False      # reference torch quantizer path
    return be


def _np(t):
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy()
    return t.numpy()


def gen_tables(out):
    lut, order, sval, bounds = ref_fp8._tables(torch.device("cpu"), torch.float32)
    out["lut"] = _np(lut)
    out["order"] = _np(order)
    out["bounds"] = _np(bounds)


def quant_cases():
    g = torch.Generator().manual_seed(20)
    sval = ref_fp8._tables(torch.device("cpu"), torch.float32)[2].tolist()
    mid = [(sval[i] + sval[i + 1]) * 0.5 for i in range(len(sval) - 1)]
    n = 16 * 256
    cases = {
        "uniform": torch.randn(16, 256, generator=g),
        "tiny": torch.randn(16, 256, generator=g) * 1e-30,
        "huge": torch.randn(16, 256, generator=g) * 1e30,
        "zeros": torch.zeros(16, 256),
        "half_zero": torch.cat([torch.zeros(8, 256), torch.randn(8, 256, generator=g)]),
        "codebook": torch.tensor((sval * 17)[:n]).view(16, 256),
        "midpoints": torch.tensor((mid * 17)[:n]).view(16, 256),
        "saturating": torch.tensor(([448.0, -448.0, 447.9, 0.0, -0.0, 1e-45] * 700)[:n]).view(16, 256),
        "subnormal": torch.randint(0, 8, (16, 256), generator=g).float() * 2.0 ** -9,
        "odd_shape": torch.randn(7, 13, generator=g),
        "padded_tile": torch.randn(5, 100, generator=g),
    }
    w = cases["saturating"].clone()
    w[0, 0] = float("nan")
    w[1, 1] = float("inf")
    w[2, 2] = float("-inf")
    cases["nonfinite"] = w
    return cases


def gen_quant(out):
    for name, w in quant_cases().items():
        out[f"q_{name}_w"] = _np(w)
        for tile in (32, 64, 128):
            import warnings
            with warnings.catch_warnings():
                warnings.simplefilter("ignore")
                codes, sc = ref_fp8.quantize_tiles(w.clone(), tile)
            out[f"q_{name}_t{tile}_codes"] = _np(codes)
            out[f"q_{name}_t{tile}_sc"] = _np(sc)


def gen_gemm(out, be):
    g = torch.Generator().manual_seed(21)
    shapes = [(33, 100, 65, 64), (64, 128, 128, 64), (96, 256, 192, 64), (5, 70, 100, 32),
              (40, 256, 64, 128), (128, 64, 64, 64)]
    out["gemm_shapes"] = np.array(shapes, dtype=np.int64)
    for i, (rows, in_f, out_f, tile) in enumerate(shapes):
        x = torch.randn(rows, in_f, generator=g)
        w32 = torch.randn(out_f, in_f, generator=g) * 0.02
        codes, sc = ref_fp8.quantize_tiles(w32, tile)
        y = be.fp8_forward(x, codes, sc, in_f, out_f, tile)
        out[f"gemm{i}_x"] = _np(x)
        out[f"gemm{i}_w"] = _np(codes)
        out[f"gemm{i}_s"] = _np(sc)
        out[f"gemm{i}_y"] = _np(y)


def _set_fp8(lin, w32, tile):
    codes, sc = ref_fp8.quantize_tiles(w32, tile)
    with torch.no_grad():
        lin.w8.copy_(codes)
        lin.sc.copy_(sc)


def _moe_case(out, tag, d, E, k, shape, dtype, seed, gate_override=None, x_override=None):
    torch.manual_seed(seed)
    cfg = ref_model.LinearConfig(vocab_size=64, d_model=d, n_layer=1, n_heads=4, is_moe=True,
                                 num_experts=E, num_experts_per_tok=k, precision="fp8",
                                 architecture="plain")
    moe = ref_model.SwiFFN_MoE(cfg).eval()
    g = torch.Generator().manual_seed(seed + 1000)
    with torch.no_grad():
        gw = gate_override if gate_override is not None else torch.randn(E, d, generator=g) * 0.02 * 8
        moe.gate.weight.copy_(gw)
        for e, ex in enumerate(moe.experts):
            for nm in ("gate", "up", "down"):
                lin = getattr(ex, nm)
                _set_fp8(lin, torch.randn(lin.out_f, lin.in_f, generator=g) * 0.02, cfg.tile)
    x = x_override if x_override is not None else torch.randn(*shape, d, generator=g)
    x = x.to(dtype)
    with torch.no_grad():
        y = moe(x)
    out[f"{tag}_meta"] = np.array([d, E, k, cfg.tile, int(moe.experts[0].gate.out_f)], dtype=np.int64)
    out[f"{tag}_dtype"] = np.array([0 if dtype == torch.float32 else 1], dtype=np.int64)
    out[f"{tag}_x"] = _np(x)
    out[f"{tag}_gate_w"] = _np(moe.gate.weight)
    for e, ex in enumerate(moe.experts):
        for nm in ("gate", "up", "down"):
            lin = getattr(ex, nm)
            out[f"{tag}_e{e}_{nm}_w"] = _np(lin.w8)
            out[f"{tag}_e{e}_{nm}_s"] = _np(lin.sc)
    out[f"{tag}_out"] = _np(y)
    out[f"{tag}_prob"] = _np(moe.last_prob)
    out[f"{tag}_topi"] = _np(moe.last_topi)
    out[f"{tag}_counts"] = np.array(moe.expert_token_counts, dtype=np.int64)
    out[f"{tag}_executed"] = np.array(moe.last_executed, dtype=np.int64)


def gen_moe(out):
    _moe_case(out, "moe_e4k2_f32", 64, 4, 2, (2, 16), torch.float32, 1)
    _moe_case(out, "moe_e4k2_bf16", 64, 4, 2, (2, 16), torch.bfloat16, 2)
    _moe_case(out, "moe_e8k3_bf16", 64, 8, 3, (1, 40), torch.bfloat16, 3)
    _moe_case(out, "moe_e8k2_bf16", 64, 8, 2, (3, 33), torch.bfloat16, 4)
    # Exact ties: all-zero router -> every probability is 1/E.
    _moe_case(out, "moe_tie_uniform", 64, 4, 2, (1, 8), torch.bfloat16, 5,
              gate_override=torch.zeros(4, 64))
    # Logits set through x[...,0] = 1 and W[:,0] = logit: a three-way tie at
    # the top and a zero-probability tail selected by k=3 (weight 0 -> not
    # dispatched, model.py:576).
    d = 64
    x = torch.zeros(1, 4, d)
    x[..., 0] = 1.0
    gw = torch.zeros(8, d)
    gw[:, 0] = torch.tensor([1.0, 1.0, -200.0, 1.0, -200.0, 0.5, -200.0, -200.0])
    _moe_case(out, "moe_tie_underflow", d, 8, 3, (1, 4), torch.float32, 6,
              gate_override=gw, x_override=x)
    gw2 = torch.zeros(8, d)
    gw2[:, 0] = torch.tensor([5.0, -200.0, -200.0, -200.0, 0.0, -200.0, -200.0, -200.0])
    _moe_case(out, "moe_zero_weight", d, 8, 3, (1, 4), torch.float32, 7,
              gate_override=gw2, x_override=x.clone())


def main():
    be = _backend()
    out = {}
    gen_tables(out)
    gen_quant(out)
    gen_gemm(out, be)
    gen_moe(out)
    path = os.path.join(HERE, "golden_fp8_moe.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
