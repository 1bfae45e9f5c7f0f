"""GPU parity of the linear-attention recurrence and of the whole C1-shaped model.

attn_forward / attn_step (the backend entries of kernel/compute.py:265-309)
run attn.hip on the device.  Bar: bit-identical to the reference kernel
kernel/attn_cpu.cpp -- here to the oracle's C restatement, which the CPU
tests pin bit-exact against that kernel and its golden vectors.

The model test runs the reference SmaulLinear's forward, prefill and step at
a config-1 shape (2 layers) through the rocm backend (tests/_model.py) and
compares with the reference model's own outputs (golden_model_c1.npz).  The
trunk runs in bf16, so every fp32 summation order that differs from the
reference's turns into bf16 rounding flips and, now and then, a routing flip.
The fixture measures that floor on the reference itself: summing its fp8 GEMM
in another valid order moves its logits by rel-L2 5.3e-3 and flips the
routing of 0.6 % of the tokens in layer 1.  The bar is twice that floor, and
at least 99 % routing agreement per layer.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from smaulnative_amd.compute import get_backend

pytestmark = pytest.mark.gpu

DEV = "cuda"
HERE = os.path.dirname(os.path.abspath(__file__))


def be():
    b = get_backend("rocm")
    assert b.has_native and b.has_attn_native
    return b


def attn_inputs(B, T, H, D, seed):
    gen = torch.Generator().manual_seed(seed)
    Q = torch.nn.functional.elu(torch.randn(B, T, H, D, generator=gen)) + 1
    K = torch.nn.functional.elu(torch.randn(B, T, H, D, generator=gen)) + 1
    V = torch.randn(B, T, H, D, generator=gen)
    return Q, K, V


@pytest.mark.parametrize("B,T,H,D", [
    (2, 256, 8, 64),    # config 1: d=512, 8 heads
    (1, 37, 3, 13),     # ragged D, partial last chunk of 16 steps
    (2, 100, 2, 128),   # the widest register-resident head (presets up to 2048/16)
    (1, 1, 4, 64),
    (1, 20, 1, 200),    # D > 128: the state in global memory
    (3, 7, 2, 1),
])
def test_attn_forward_bit_exact(B, T, H, D):
    print(f"case attn_forward B={B} T={T} H={H} D={D}", flush=True)
    Q, K, V = attn_inputs(B, T, H, D, B * 7 + T * 3 + D)
    Yr, DENr, Sr, zr = oracle.attn_forward(Q, K, V)
    Y, DEN, S, z = be().attn_forward(Q.to(DEV), K.to(DEV), V.to(DEV), 1e-6, True, need_state=True)
    torch.cuda.synchronize()
    assert torch.equal(Y.cpu(), Yr)
    assert torch.equal(DEN.cpu(), DENr)
    assert torch.equal(S.cpu(), Sr) and torch.equal(z.cpu(), zr)
    # without DEN and state: the same Y, zero-element placeholders (compute.py:265-289)
    Y2, DEN2, S2, z2 = be().attn_forward(Q.to(DEV), K.to(DEV), V.to(DEV), 1e-6, False)
    assert DEN2 is None and S2.numel() == 0 and z2.numel() == 0
    assert torch.equal(Y2.cpu(), Yr)


def test_attn_forward_empty_and_zero_keys():
    # T = 0 with the state requested: zeros (attn_cpu.cpp:176-188)
    Q, K, V = attn_inputs(2, 0, 3, 64, 1)
    Y, DEN, S, z = be().attn_forward(Q.to(DEV), K.to(DEV), V.to(DEV), 1e-6, True, need_state=True)
    assert Y.shape == Q.shape and tuple(S.shape) == (2, 3, 64, 64)
    assert float(S.abs().sum()) == 0.0 and float(z.abs().sum()) == 0.0
    # all-zero keys: the 1e-6 norm clamp, den clamped to eps, y = 0
    Q, K, V = attn_inputs(1, 5, 2, 32, 2)
    K[:, 2] = 0.0
    Yr, DENr, Sr, zr = oracle.attn_forward(Q, K, V)
    Y, DEN, S, z = be().attn_forward(Q.to(DEV), K.to(DEV), V.to(DEV), 1e-6, True, need_state=True)
    assert torch.equal(Y.cpu(), Yr) and torch.equal(DEN.cpu(), DENr) and torch.equal(S.cpu(), Sr)


@pytest.mark.parametrize("B,H,D", [(2, 8, 64), (1, 3, 13), (1, 2, 300)])
def test_attn_step_bit_exact_and_chains(B, H, D):
    """attn_step advances (S, z) in place, bit-identical to the reference step;
    prefill over T-3 tokens then 3 steps equals the forward over T tokens."""
    print(f"case attn_step B={B} H={H} D={D}", flush=True)
    T = 24
    Q, K, V = attn_inputs(B, T, H, D, D + H)
    Yr = oracle.attn_forward(Q, K, V)[0]
    b = be()
    _, _, S, z = b.attn_forward(Q[:, :-3].to(DEV), K[:, :-3].to(DEV), V[:, :-3].to(DEV), 1e-6, False,
                                need_state=True)
    Sc, zc = S.cpu(), z.cpu()
    for t in range(T - 3, T):
        q, k, v = (X[:, t].contiguous() for X in (Q, K, V))
        yo, Sc, zc = oracle.attn_step(Sc, zc, q, k, v)
        y, S2, z2 = b.attn_step(S, z, q.to(DEV), k.to(DEV), v.to(DEV), 1e-6)
        assert S2.data_ptr() == S.data_ptr() and z2.data_ptr() == z.data_ptr()  # in place
        torch.cuda.synchronize()
        assert torch.equal(y.cpu(), yo)
        assert torch.equal(S.cpu(), Sc) and torch.equal(z.cpu(), zc)
        assert torch.equal(y.cpu(), Yr[:, t])


def test_attn_golden_vectors():
    """The vectors written from the reference's attn_cpu.cpp, on the device."""
    ga = np.load(os.path.join(HERE, "golden", "golden_attn.npz"))
    b = be()
    for i, eps in enumerate(ga["eps"].tolist()):
        g = {k[len(f"a{i}_"):]: torch.from_numpy(ga[k]) for k in ga.files if k.startswith(f"a{i}_")}
        print(f"case golden attn {i} shape {tuple(g['Q'].shape)} eps {eps}", flush=True)
        Y, DEN, S, z = b.attn_forward(g["Q"].to(DEV), g["K"].to(DEV), g["V"].to(DEV), eps, True, need_state=True)
        assert torch.equal(Y.cpu(), g["Y"]) and torch.equal(DEN.cpu(), g["DEN"]) and torch.equal(z.cpu(), g["z"])
        if "S" in g:
            assert torch.equal(S.cpu(), g["S"])
        y1, S, z = b.attn_step(S, z, g["q"].to(DEV), g["k"].to(DEV), g["v"].to(DEV), eps)
        assert torch.equal(y1.cpu(), g["y1"]) and torch.equal(z.cpu(), g["z1"])
        if "S1" in g:
            assert torch.equal(S.cpu(), g["S1"])


def test_attn_rejects_bad_inputs():
    b = be()
    Q, K, V = (t.to(DEV) for t in attn_inputs(1, 4, 2, 8, 3))
    with pytest.raises(RuntimeError, match="float32"):
        b.attn_forward(Q.double(), K, V, 1e-6, False)
    with pytest.raises(RuntimeError, match="eps"):
        b.attn_forward(Q, K, V, 0.0, False)
    with pytest.raises(RuntimeError, match="HIP device"):
        b.attn_forward(Q.cpu(), K.cpu(), V.cpu(), 1e-6, False)
    _, _, S, z = b.attn_forward(Q, K, V, 1e-6, False, need_state=True)
    with pytest.raises(RuntimeError, match="contiguous"):
        b.attn_step(S.transpose(2, 3), z, Q[:, 0], K[:, 0], V[:, 0], 1e-6)


def test_model_c1_forward_prefill_step_vs_reference():
    """The reference SmaulLinear (config 1 cut to 2 layers) through the rocm backend."""
    from _model import Trunk, draw_state
    from smaulnative_amd.fp8_tile import quantize_tiles
    g = np.load(os.path.join(HERE, "golden", "golden_model_c1.npz"))
    sd, idx = draw_state(quantize_tiles)
    assert np.array_equal(idx.numpy(), g["idx"])
    m = Trunk(sd, torch.device(DEV))
    logits, topi = m.forward(idx)
    pos = g["positions"].tolist()
    got = logits[:, pos].cpu().double()
    ref = torch.from_numpy(g["forward_logits"]).double()
    err = float((got - ref).norm() / ref.norm())
    agree = [float((t.cpu() == torch.from_numpy(g[f"layer{l}_topi"])).all(-1).float().mean())
             for l, t in enumerate(topi)]
    floor = float(g["reorder_rel_l2"])
    print(f"forward logits rel_l2 {err:.3e} (reference reorder floor {floor:.3e}); routing agreement per "
          f"layer {agree} (reference reorder {g['reorder_routing_agreement'].tolist()})", flush=True)
    assert err < 2 * floor
    assert min(agree) >= 0.99
    pl, states = m.prefill(idx[:, :-1])
    sl, _ = m.step(idx[:, -1:], states)
    for name, a, r in (("prefill", pl, g["prefill_logits"]), ("step", sl, g["step_logits"])):
        r = torch.from_numpy(r).double()
        e = float((a.cpu().double() - r).norm() / r.norm())
        print(f"{name} logits rel_l2 {e:.3e}", flush=True)
        assert e < 2 * floor


@pytest.mark.parametrize("layer", [0, 1])
def test_model_c1_moe_layer_on_reference_inputs(layer):
    """Each config-1 MoE layer on the reference model's own input: the exact
    bf16 x its Block handed to self.ffn (model.py:646), through SwiFFN_MoE on
    the rocm backend.  Routing bit-exact (top-k and counts equal), last_prob
    within 1e-5 relative, output within rel-L2 2e-3 of the reference layer's
    fx (golden_model_c1.npz)."""
    from test_oracle import c1_layer_case
    from smaulnative_amd import MoEConfig, SwiFFN_MoE
    from _model import C1
    print(f"case C1 MoE layer {layer} on the reference's inputs", flush=True)
    x, gw, experts, fx, prob, topi, counts = c1_layer_case(layer)
    moe = SwiFFN_MoE(MoEConfig(d_model=C1["d"], ffn_mult=C1["ffn_mult"], tile=C1["tile"],
                               num_experts=C1["experts"], num_experts_per_tok=C1["top_k"]))
    with torch.no_grad():
        moe.gate.weight.copy_(gw)
        for e, ex in enumerate(moe.experts):
            for n in ("gate", "up", "down"):
                getattr(ex, n).w8.copy_(getattr(experts[e], n + "_w"))
                getattr(ex, n).sc.copy_(getattr(experts[e], n + "_s"))
    moe = moe.to(DEV).eval()
    with torch.no_grad():
        y = moe(x.reshape(C1["batch"], C1["ctx"], -1).to(DEV))
    got_topi = moe.last_topi.reshape(-1, C1["top_k"]).cpu()
    assert torch.equal(got_topi, topi), int((got_topi != topi).any(-1).sum())
    assert moe.expert_token_counts == counts
    p = moe.last_prob.reshape(-1, C1["experts"]).cpu().double()
    assert float(((p - prob.double()).abs() / prob.double().abs().clamp_min(1e-30)).max()) < 1e-5
    y = y.reshape(-1, C1["d"]).cpu().double()
    err = float((y - fx.double()).norm() / fx.double().norm())
    print(f"layer {layer}: routing bit-exact, rel_l2 {err:.3e}", flush=True)
    assert err <= 2e-3


@pytest.mark.parametrize("B,T,H,D,eps", [(2, 37, 3, 64, 1e-6), (1, 5, 2, 13, 1e-6), (1, 24, 2, 128, 1e-6),
                                         (1, 3, 1, 200, 1e-6), (1, 40, 1, 7, 1e-6), (1, 1, 1, 1, 1e-6),
                                         (2, 19, 2, 100, 50.0)])
def test_attn_backward_bit_exact_vs_oracle(B, T, H, D, eps):
    """attn_backward on the device (kernel/attn_cpu.cpp:227-368 restated) equals
    the oracle bit for bit: the state in LDS (D <= 64, D <= 128) and in the
    workspace (D = 200), remainders of the 8-lane sums (D = 13, 7, 1, 100),
    every den clamped (eps = 50)."""
    print(f"case attn_backward B={B} T={T} H={H} D={D} eps={eps}", flush=True)
    Q, K, V = attn_inputs(B, T, H, D, B * 31 + T * 7 + D)
    if D == 13:
        K[:, 1] = 0.0  # zero keys: the 1e-6 clamp and the guarded nc^3 division
    dY = torch.randn(B, T, H, D, generator=torch.Generator().manual_seed(T + D))
    Y, DEN, _, _ = oracle.attn_forward(Q, K, V, eps)
    ref = oracle.attn_backward(dY, Q, K, V, Y, DEN, eps)
    got = be().attn_backward(*(t.to(DEV) for t in (dY, Q, K, V, Y, DEN)), eps)
    torch.cuda.synchronize()
    for name, a, r in zip(("dQ", "dK", "dV"), got, ref):
        assert torch.equal(a.cpu(), r), name


def test_attn_backward_without_den_reruns_forward():
    """With DEN missing (the reference then falls back to autograd through its
    torch recurrence), the backend reruns the forward on the device for it:
    the same bits as with the forward's DEN."""
    Q, K, V = (t.to(DEV) for t in attn_inputs(1, 9, 2, 32, 77))
    dY = torch.randn_like(Q)
    Y, DEN = be().attn_forward(Q, K, V, 1e-6, True)[:2]
    a = be().attn_backward(dY, Q, K, V, Y, DEN, 1e-6)
    b = be().attn_backward(dY, Q, K, V, Y, None, 1e-6)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x.cpu(), y.cpu())


class _AttnFn(torch.autograd.Function):
    """model.py:235-265 (_LinearAttnFn): the backend's attn_forward with DEN,
    its attn_backward for the gradients."""

    @staticmethod
    def forward(ctx, Q, K, V, eps):
        Y, DEN = be().attn_forward(Q, K, V, eps, True)[:2]
        ctx.save_for_backward(Q, K, V, Y, DEN)
        ctx.eps = eps
        return Y

    @staticmethod
    def backward(ctx, dY):
        Q, K, V, Y, DEN = ctx.saved_tensors
        return (*be().attn_backward(dY.contiguous(), Q, K, V, Y, DEN, ctx.eps), None)


def test_training_block_step_on_device():
    """A training-mode step of one config-1-shaped Block (model.py:624-649: the
    q/k/v/o FP8Linear projections, the elu+1 features, the linear-attention
    recurrence, the RMSNorms and the SwiFFN_MoE) with autograd, every kernel
    on rocm: the attention forward and backward, the FP8 GEMMs and their input
    gradients, the MoE training path.  Checked against autograd of a float64
    restatement on the decoded weights with the same routing: output and
    input gradient within rel-L2 2e-2 (bf16 activations; measured 6e-3 and
    7e-3), every projection
    and executed expert accumulating _gw, the router gradient finite."""
    import torch.nn.functional as F
    from smaulnative_amd import FP8Linear, MoEConfig, SwiFFN_MoE
    from smaulnative_amd.fp8_tile import decode_block
    print("case training block step on the device", flush=True)
    torch.manual_seed(3)
    d, Hh, E, k = 128, 2, 4, 2
    D = d // Hh
    proj = {n: FP8Linear(d, d, 64).to(DEV).train() for n in ("q", "k", "v", "o")}
    moe = SwiFFN_MoE(MoEConfig(d_model=d, ffn_mult=2.5, tile=64, num_experts=E, num_experts_per_tok=k)).to(DEV)
    moe.train()
    nw = [(1.0 + 0.1 * torch.randn(d)).to(DEV) for _ in range(5)]
    x0 = torch.randn(2, 48, d, device=DEV).to(torch.bfloat16)
    c = torch.randn(2, 48, d, device=DEV)

    def block(x, lin, attn, ffn, dt, ft):
        # dt: the activation dtype (bf16; float64 in the restatement), ft: the
        # dtype of the fp32 points (.float() in model.py; float64 there too)
        def rms(t, w):
            tf = t.to(ft)
            return (tf * torch.rsqrt(tf.pow(2).mean(-1, keepdim=True) + 1e-6) * w.to(ft)).to(t.dtype)
        B, T, _ = x.shape
        n1x = rms(x, nw[0])
        q = F.elu(lin("q", n1x).to(ft).view(B, T, Hh, D)) + 1.0
        kk = F.elu(lin("k", n1x).to(ft).view(B, T, Hh, D)) + 1.0
        v = lin("v", n1x).to(ft).view(B, T, Hh, D)
        y = attn(q, kk, v).reshape(B, T, d)
        ax = lin("o", y.to(dt))
        a = rms(ax.to(ft), nw[1])
        x = rms((x.to(ft) + a.to(ft)).to(dt), nw[2])
        fx = ffn(x)
        f = rms(fx.to(ft), nw[3])
        return rms((x.to(ft) + f.to(ft)).to(dt), nw[4])

    x = x0.clone().requires_grad_(True)
    out = block(x, lambda n, t: proj[n](t), lambda q, kk, v: _AttnFn.apply(q.contiguous(), kk.contiguous(),
                                                                            v.contiguous(), 1e-6),
                moe, torch.bfloat16, torch.float32)
    (out.float() * c).sum().backward()
    topi = moe.last_topi.reshape(-1, k)
    assert all(proj[n]._gw is not None for n in proj)
    assert torch.isfinite(moe.gate.weight.grad).all()
    for e, cnt in enumerate(moe.expert_token_counts):
        assert (moe.experts[e].gate._gw is not None) == (cnt > 0)

    # float64 restatement: decoded weights, the textbook recurrence, the same routing
    def dense(m):
        return decode_block(m.w8, m.sc, 0, m.out_f, m.in_f, m.tile).double()
    W = {n: dense(proj[n]) for n in proj}
    gw = moe.gate.weight.detach().double()
    EW = [{n: dense(getattr(ex, n)) for n in ("gate", "up", "down")} for ex in moe.experts]

    def attn64(q, kk, v):
        B, T = q.shape[:2]
        S = torch.zeros(B, Hh, D, D, dtype=torch.float64, device=DEV)
        z = torch.zeros(B, Hh, D, dtype=torch.float64, device=DEV)
        ys = []
        for t in range(T):
            kt = kk[:, t] / kk[:, t].norm(dim=-1, keepdim=True).clamp_min(1e-6)
            S = S + kt.unsqueeze(-1) @ v[:, t].unsqueeze(-2)
            z = z + kt
            ys.append((q[:, t].unsqueeze(-2) @ S).squeeze(-2) / (q[:, t] * z).sum(-1, keepdim=True).clamp_min(1e-6))
        return torch.stack(ys, 1)

    def ffn64(xm):
        xs = xm.reshape(-1, d)
        prob = torch.softmax(xs @ gw.t(), -1)
        topv = prob.gather(-1, topi)
        topv = topv / topv.sum(-1, keepdim=True)
        o = torch.zeros_like(xs)
        for e in range(E):
            w = torch.where(topi == e, topv, torch.zeros_like(topv)).sum(-1)
            rows = torch.nonzero(w > 0).squeeze(-1)
            if rows.numel():
                h = F.silu(xs[rows] @ EW[e]["gate"].t()) * (xs[rows] @ EW[e]["up"].t())
                o = o.index_add(0, rows, (h @ EW[e]["down"].t()) * w[rows].unsqueeze(-1))
        return o.view(xm.shape)

    xr = x0.detach().double().requires_grad_(True)
    ref = block(xr, lambda n, t: t.double() @ W[n].t(), attn64, ffn64, torch.float64, torch.float64)
    (ref * c.double()).sum().backward()

    def rel(a, b):
        return float((a.double() - b).norm() / b.norm())
    e_out, e_dx = rel(out.detach(), ref.detach()), rel(x.grad, xr.grad)
    print(f"block step: out rel_l2 {e_out:.2e}, x.grad rel_l2 {e_dx:.2e}", flush=True)
    assert e_out < 2e-2 and e_dx < 2e-2
