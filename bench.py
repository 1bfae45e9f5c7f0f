#!/usr/bin/env python3
"""MoE-layer benchmark on one MI355X (BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-decode]

Headline (``value``): tokens/s of one SmaulMoE layer at config 3 -- prefill,
T=16384 tokens, d=1024, expert hidden h=2560, E=8 experts, top-2, tile 64,
bf16 activations, router bias N(0, 0.5).  A step is one full layer forward
(router -> dispatch -> gate/up SwiGLU grouped GEMM -> down grouped GEMM ->
combine) over inputs already resident in HBM.

Extra objects on the same JSON line:
- ``roofline``: the dominant kernel (the gate/up grouped GEMM), algorithmic
  FLOPs per launch / its mean duration from HIP events on the launch stream,
  against the bf16 dense MFMA peak;
- ``cpu_baseline``: the reference CPU path on this host's cores -- the
  reference's own fp8_cpu.cpp (built under oracle/_ref) inside the torch MoE
  loop of model.py:557-585 -- on a bounded sample of the same tokens;
- ``decode``: config 4 (64 tokens x 24 MoE layers), one step replayed as a HIP
  graph, with achieved HBM bytes/s against the 8 TB/s peak.
Only one GPU is measured: ``--gpus`` above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

PEAK_BF16_FLOPS = 2.5e15    # MI355X dense bf16 MFMA
PEAK_HBM_BPS = 8.0e12       # MI355X HBM3E
METRIC = "MoE-layer tokens/s + % bf16 MFMA peak (prefill), % HBM BW (decode), 1 GPU"
HERE = os.path.dirname(os.path.abspath(__file__))


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_layer(seed, T, d, h, E, bias_std, device, gen_device="cpu"):
    """Config-3 style synthetic layer: x, router W/b, E experts as tiled E4M3.

    Draw order (one generator): x, router W, router b, then per expert the
    gate, up and down weights, each N(0, 0.02).
    """
    import torch
    from smaulnative_amd.fp8_tile import quantize_tiles
    gen = torch.Generator(device=gen_device).manual_seed(seed)
    x = torch.randn(T, d, generator=gen, device=gen_device)
    gw = torch.randn(E, d, generator=gen, device=gen_device) * 0.02
    gb = torch.randn(E, generator=gen, device=gen_device) * bias_std
    experts = []
    for _ in range(E):
        parts = []
        for (o, i) in ((h, d), (h, d), (d, h)):
            w8, sc = quantize_tiles(torch.randn(o, i, generator=gen, device=gen_device) * 0.02, 64)
            parts += [w8, sc]
        experts.append(tuple(parts))
    return x.to(torch.bfloat16), gw, gb, experts


def time_prefill(be, xd, gwd, gbd, exd, k, steps, warmup):
    import torch
    for _ in range(warmup):
        be.moe_forward(xd, gwd, gbd, exd, k, 64)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = be.moe_forward(xd, gwd, gbd, exd, k, 64)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return (t1 - t0) / steps, out


def time_stages(be, xd, gwd, gbd, exd, k, steps):
    """Mean per-stage device time from HIP events on the launch stream."""
    import torch
    names = ["router", "dispatch", "gate_up", "down", "combine"]
    acc = [0.0] * 5
    for it in range(steps + 2):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(6)]
        be.moe_stages(xd, gwd, gbd, exd, k, 64, events=ev)
        torch.cuda.synchronize()
        if it >= 2:
            for i in range(5):
                acc[i] += ev[i].elapsed_time(ev[i + 1])
    return {n: a / steps for n, a in zip(names, acc)}


def cpu_baseline(x, gw, gb, experts, k, target_s=10.0):
    """Reference CPU path on a bounded token sample (tokens are independent)."""
    import torch
    import oracle
    cores = oracle.default_threads()
    torch.set_num_threads(cores)
    os.environ["OMP_NUM_THREADS"] = str(cores)
    ref = oracle.ref_module()
    gemm = oracle.fp8_forward_ref if ref is not None else (
        lambda xx, w, s, i, o, t: oracle.fp8_forward(xx, w, s, i, o, t, threads=cores))
    kind = "reference" if ref is not None else "port"
    ow = [oracle.ExpertWeights(*e) for e in experts]
    oracle.moe_forward(x[:64], gw, gb, ow, k, 64, gemm=gemm)  # warm-up
    n = 512
    t0 = time.perf_counter()
    oracle.moe_forward(x[:n], gw, gb, ow, k, 64, gemm=gemm)
    dt = time.perf_counter() - t0
    if dt < target_s / 4 and n < x.shape[0]:
        n = int(min(x.shape[0], max(n, n * target_s / max(dt, 1e-3))))
        t0 = time.perf_counter()
        oracle.moe_forward(x[:n], gw, gb, ow, k, 64, gemm=gemm)
        dt = time.perf_counter() - t0
    what = ("reference kernel/fp8_cpu.cpp (oracle/_ref) in the model.py:557-585 torch MoE loop"
            if kind == "reference" else "C restatement of fp8_cpu.cpp in the model.py:557-585 MoE loop")
    return {"value": n / dt, "unit": "tokens/s", "cores": cores, "kind": kind,
            "sample": f"first {n} of the config-3 tokens, one pass, {dt:.2f} s; {what}"}


def decode_bench(be, steps, warmup, layers=24, T=64, d=1024, h=2560, E=8, k=2):
    """Config 4: 64 tokens through 24 stacked MoE layers (independent weights, each
    layer fed the unit-RMS-normalised output of the one before), one HIP graph
    replay per step."""
    import torch
    dev = torch.device("cuda")
    lay = []
    for l in range(layers):
        x, gw, gb, ex = make_layer(4000 + l, T, d, h, E, 0.5, dev, gen_device="cuda")
        lay.append((gw.to(dev), gb.to(dev), [tuple(t.to(dev) for t in e) for e in ex]))
    x0 = torch.randn(T, d, generator=torch.Generator(device="cuda").manual_seed(1237),
                     device=dev).to(torch.bfloat16)
    x0 = (x0.float() * torch.rsqrt(x0.float().pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)

    def step(chained=True):
        # layer l + 1 reads layer l's output after a unit-RMS row norm (Block's
        # norm around the FFN, model.py:636), so the 24 layers form one chain;
        # chained: layer l + 1's router runs inside layer l's combine + norm
        outs = []
        xl = x0
        routing = None
        for l, (gw, gb, ex) in enumerate(lay):
            nr = (lay[l + 1][0], lay[l + 1][1], k) if chained and l + 1 < layers else None
            o = be.moe_forward_norm(xl, gw, gb, ex, k, 64, None, 1e-6, routing=routing, next_router=nr)
            outs.append(o)
            xl = o[4]
            routing = o[5] if nr is not None else None
        return outs

    eager = step()
    plain = step(False)
    torch.cuda.synchronize()
    chain_ok = all(torch.equal(a[0], b[0]) and torch.equal(a[4], b[4]) for a, b in zip(eager, plain))
    del plain
    counts = [o[3].cpu() for o in eager]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()  # warm the caches of the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            gouts = step()
    torch.cuda.synchronize()
    for _ in range(max(1, warmup)):
        g.replay()
    torch.cuda.synchronize()
    ok = all(torch.equal(a[0], b[0]) for a, b in zip(eager, gouts))
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    # eager (no graph) for reference
    t0 = time.perf_counter()
    for _ in range(max(1, steps // 4)):
        step()
    torch.cuda.synchronize()
    dt_eager = (time.perf_counter() - t0) / max(1, steps // 4)
    expert_bytes = 3 * d * h * (1 + 4 / 64)
    nbytes = 0.0
    for c in counts:
        executed = int((c > 0).sum())
        nbytes += executed * expert_bytes + 4 * E * d + 2 * T * d * 2
    return {"workload": "C4 decode: 64 tokens x 24 chained MoE layers (unit-RMS norm between layers, each "
                        "layer's router fused into the previous layer's combine + norm), d=1024 h=2560 E=8 "
                        "top-2, HIP graph replay",
            "tokens_per_s": T / dt, "ms_per_step": dt * 1e3, "ms_per_step_eager": dt_eager * 1e3,
            "bytes_per_step": nbytes, "hbm_GBps": nbytes / dt / 1e9,
            "hbm_frac": nbytes / dt / PEAK_HBM_BPS, "graph_matches_eager": ok,
            "chain_matches_unfused": chain_ok}


def read_traffic():
    """HBM bytes per gate_up launch from the committed rocprofv3 --pmc summary, if any."""
    p = os.path.join(HERE, "profiles", "gate_up_c3_traffic.txt")
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1].strip())
            except ValueError:
                return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run 3 device-to-device copies of BYTES (calibrates rocprofv3 "
                         "FETCH_SIZE/WRITE_SIZE against a kernel of known traffic), then exit")
    args = ap.parse_args()
    if args.copy_probe:
        import torch
        src = torch.ones(args.copy_probe // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": src.numel() * 4}), flush=True)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}, "
              f"WORLD_SIZE={world}", file=sys.stderr)
        sys.exit(2)

    import torch
    sys.path.insert(0, HERE)
    from smaulnative_amd.compute import get_backend
    be = get_backend("rocm")
    if not be.has_native:
        raise SystemExit("libsmaul_rocm.so is not built")
    dev = torch.device("cuda")

    T, d, h, E, k = 16384, 1024, 2560, 8, 2
    log("bench: building config-3 workload")
    x, gw, gb, experts = make_layer(1236, T, d, h, E, 0.5, "cpu")
    xd, gwd, gbd = x.to(dev), gw.to(dev), gb.to(dev)
    exd = [tuple(t.to(dev) for t in e) for e in experts]

    log("bench: timing prefill layer")
    sec, out = time_prefill(be, xd, gwd, gbd, exd, k, args.steps, args.warmup)
    counts = out[3].cpu().tolist()
    stages = time_stages(be, xd, gwd, gbd, exd, k, max(3, args.steps // 2))
    log("bench: stages ms", {kk: round(v, 4) for kk, v in stages.items()})
    R = T * k
    flops_router = 2.0 * T * d * E
    flops_gate_up = 2.0 * R * d * (2 * h)
    flops_down = 2.0 * R * h * d
    total_flops = flops_router + flops_gate_up + flops_down
    gu_s = stages["gate_up"] * 1e-3
    roof = {"kernel": "fp8_gemm_dma_kernel (gate_up, SwiGLU epilogue)", "bound": "mfma",
            "achieved": flops_gate_up / gu_s / 1e12, "peak": PEAK_BF16_FLOPS / 1e12, "unit": "TFLOP/s",
            "frac": flops_gate_up / gu_s / PEAK_BF16_FLOPS, "traffic": read_traffic(),
            "flops_per_launch": flops_gate_up, "mean_launch_ms": stages["gate_up"]}
    res = {
        "metric": METRIC,
        "value": T / sec,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sec * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) activations (cast to bf16 once), N(0,0.02) weights quantized to "
                "tiled E4M3 (tile 64), router bias N(0,0.5)",
        "config": {"workload": "C3 MoE prefill: one SwiFFN_MoE layer, T=16384 d=1024 h=2560 E=8 top-2 tile=64",
                   "tokens": T, "d_model": d, "hidden": h, "experts": E, "top_k": k,
                   "expert_token_counts": counts},
        "layer_mfma_frac": total_flops / sec / PEAK_BF16_FLOPS,
        "layer_tflops": total_flops / sec / 1e12,
        "stages_ms": stages,
        "roofline": roof,
    }
    if not args.no_decode:
        log("bench: decode (config 4)")
        try:
            res["decode"] = decode_bench(be, max(5, args.steps), args.warmup)
        except Exception as exc:  # report, keep the headline
            res["decode"] = {"error": f"{type(exc).__name__}: {exc}"}
    if not args.no_cpu:
        log("bench: CPU baseline")
        try:
            res["cpu_baseline"] = cpu_baseline(x, gw, gb, experts, k)
        except Exception as exc:
            res["cpu_baseline"] = {"error": f"{type(exc).__name__}: {exc}"}
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
