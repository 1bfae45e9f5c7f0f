"""Pins the CPU oracle before anything is checked against it.

Every function of oracle/ is checked here against (a) the golden vectors in
tests/golden/ written from the reference itself (tests/golden/make_golden.py),
(b) the reference's own fp8_cpu.cpp built under oracle/_ref where present, and
(c) what the mathematics fixes (closed form of the codebook, brute-force
x @ decode(W).T).  A planted mistake in the GEMM's rounding order is shown to
fail the golden check, so the golden check can tell the two orders apart.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from _cases import load_moe_case

GOLD = os.path.join(os.path.dirname(__file__), "golden", "golden_fp8_moe.npz")


@pytest.fixture(scope="module")
def g():
    return np.load(GOLD)


def _t(a):
    return torch.from_numpy(np.array(a))


def _bf(a):
    return torch.from_numpy(np.array(a)).view(torch.bfloat16)


# --------------------------------------------------------------------------
# codebook
# --------------------------------------------------------------------------
def _closed_form(c):
    e, m = (c >> 3) & 15, c & 7
    s = -1.0 if c & 128 else 1.0
    if e == 15 and m == 7:
        return s * 448.0
    if e == 0:
        return s * m * 2.0 ** -9
    return s * (1 + m / 8.0) * 2.0 ** (e - 7)


def test_lut_closed_form_and_golden(g):
    lut = oracle.e4m3_lut()
    assert [float(v) for v in lut] == [_closed_form(c) for c in range(256)]
    assert np.array_equal(lut.view(np.uint32), g["lut"].view(np.uint32))
    assert np.array_equal(oracle.c_lut().view(np.uint32), g["lut"].view(np.uint32))
    # reference conventions: 0x7E/0x7F = 448, 0xFE/0xFF = -448, 0x80 = -0
    assert lut[0x7E] == lut[0x7F] == 448.0 and lut[0xFE] == lut[0xFF] == -448.0
    assert lut[0x80] == 0.0 and np.signbit(lut[0x80])
    # every value is exact in bf16 (3-bit mantissa, exponents 2^-9..2^8)
    as_bf = torch.from_numpy(lut).to(torch.bfloat16).float().numpy()
    assert np.array_equal(as_bf, lut)


def test_quant_tables_match_reference(g):
    _, order, _, bounds = oracle.quant_tables()
    assert np.array_equal(order.numpy(), g["order"])
    assert np.array_equal(bounds.numpy().view(np.uint32), g["bounds"].view(np.uint32))


# --------------------------------------------------------------------------
# quantizer (oracle restatement and the product's own weight-prep quantizer)
# --------------------------------------------------------------------------
QCASES = ["uniform", "tiny", "huge", "zeros", "half_zero", "codebook", "midpoints", "saturating",
          "subnormal", "odd_shape", "padded_tile", "nonfinite"]


@pytest.mark.parametrize("tile", [32, 64, 128])
@pytest.mark.parametrize("name", QCASES)
def test_quantize_matches_golden(g, name, tile):
    import warnings
    w = _t(g[f"q_{name}_w"])
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        codes, sc = oracle.quantize_tiles(w.clone(), tile)
        from smaulnative_amd.fp8_tile import quantize_tiles as prod_quantize
        pc, ps = prod_quantize(w.clone(), tile)
    assert np.array_equal(codes.numpy(), g[f"q_{name}_t{tile}_codes"])
    assert np.array_equal(sc.numpy().view(np.uint32), g[f"q_{name}_t{tile}_sc"].view(np.uint32))
    assert torch.equal(pc, codes) and torch.equal(ps, sc)


# --------------------------------------------------------------------------
# fp8 GEMM (C restatement of fp8_cpu.cpp)
# --------------------------------------------------------------------------
def test_fp8_forward_bit_exact_with_golden(g):
    for i, (rows, in_f, out_f, tile) in enumerate(g["gemm_shapes"].tolist()):
        x, w, s = _t(g[f"gemm{i}_x"]), _t(g[f"gemm{i}_w"]), _t(g[f"gemm{i}_s"])
        y = oracle.fp8_forward(x, w, s, in_f, out_f, tile)
        assert np.array_equal(y.numpy().view(np.uint32), g[f"gemm{i}_y"].view(np.uint32)), (rows, in_f, out_f)


def test_fp8_forward_matches_bruteforce():
    # test_linear_fp8.py:170-183 shapes: forward vs x @ decode(W).T, rel < 1e-5
    for in_f, out_f, rows in [(128, 64, 9), (100, 70, 5), (65, 65, 33), (512, 256, 64)]:
        torch.manual_seed(0)
        w, s = oracle.quantize_tiles(torch.randn(out_f, in_f) * 0.05, 64)
        x = torch.randn(rows, in_f)
        y = oracle.fp8_forward(x, w, s, in_f, out_f, 64)
        ref = x.double() @ oracle.decode_full(w, s, 64).double().T
        rel = float((y.double() - ref).abs().max() / ref.abs().max())
        assert rel < 1e-5, (in_f, out_f, rows, rel)


def test_fp8_forward_threads_do_not_change_bits():
    torch.manual_seed(3)
    w, s = oracle.quantize_tiles(torch.randn(200, 192) * 0.02, 64)
    x = torch.randn(77, 192)
    a = oracle.fp8_forward(x, w, s, 192, 200, 64, threads=1)
    b = oracle.fp8_forward(x, w, s, 192, 200, 64, threads=8)
    assert torch.equal(a, b)


@pytest.mark.skipif(oracle.ref_module() is None, reason="oracle/_ref (reference build) not present")
@pytest.mark.parametrize("rows,in_f,out_f,tile", [(33, 100, 65, 64), (64, 128, 128, 64), (5, 70, 100, 32),
                                                  (96, 256, 192, 128), (64, 64, 64, 16), (130, 640, 96, 64)])
def test_fp8_forward_bit_exact_with_reference_build(rows, in_f, out_f, tile):
    torch.manual_seed(rows + in_f)
    x = torch.randn(rows, in_f)
    w, s = oracle.quantize_tiles(torch.randn(out_f, in_f) * 0.02, tile)
    assert torch.equal(oracle.fp8_forward(x, w, s, in_f, out_f, tile),
                       oracle.fp8_forward_ref(x, w, s, in_f, out_f, tile))


def _numpy_gemm(x, w, s, tile, fast_order):
    """A float32 numpy GEMM with one rounding order for every K block."""
    lut = oracle.e4m3_lut()
    xs, ws, ss = x.numpy(), w.numpy(), s.numpy()
    rows, in_f = xs.shape
    out_f = ws.shape[0]
    acc = np.zeros((rows, out_f), dtype=np.float32)
    for k in range(in_f):
        col = lut[ws[:, k]]
        sk = ss[:, k // tile]
        if fast_order:
            p = xs[:, k:k + 1] * (col * sk)[None, :]
        else:
            p = (xs[:, k:k + 1] * col[None, :]) * sk[None, :]
        acc = (acc + p.astype(np.float32)).astype(np.float32)
    return acc


def test_golden_gemm_distinguishes_rounding_orders(g):
    # golden shape 1 is 64x128 -> 128: every task is on the reference's fast
    # path, x*(lut*s).  The planted mistake (x*lut)*s must NOT reproduce it.
    i = 1
    x, w, s = _t(g[f"gemm{i}_x"]), _t(g[f"gemm{i}_w"]), _t(g[f"gemm{i}_s"])
    good = _numpy_gemm(x, w, s, 64, fast_order=True)
    bad = _numpy_gemm(x, w, s, 64, fast_order=False)
    gold = g[f"gemm{i}_y"]
    assert np.array_equal(good.view(np.uint32), gold.view(np.uint32))
    assert not np.array_equal(bad.view(np.uint32), gold.view(np.uint32))


# --------------------------------------------------------------------------
# MoE forward (router, top-k ties, w>0 mask, combine order, dtype rounding)
# --------------------------------------------------------------------------
MOE_CASES = ["moe_e4k2_f32", "moe_e4k2_bf16", "moe_e8k3_bf16", "moe_e8k2_bf16", "moe_tie_uniform",
             "moe_tie_underflow", "moe_zero_weight"]


@pytest.mark.parametrize("tag", MOE_CASES)
def test_moe_oracle_matches_golden(g, tag):
    c = load_moe_case(g, tag)
    r = oracle.moe_forward(c["x"], c["gate_w"], None, c["experts"], c["k"], c["tile"])
    assert torch.equal(r.topi, c["topi"]), tag
    assert r.counts == c["counts"] and r.executed == c["executed"]
    assert torch.equal(r.prob, c["prob"]), tag
    assert torch.equal(r.out.view(torch.int16) if r.out.dtype == torch.bfloat16 else r.out,
                       c["out"].view(torch.int16) if c["out"].dtype == torch.bfloat16 else c["out"]), tag


def test_moe_oracle_perm_is_ascending_and_complete(g):
    c = load_moe_case(g, "moe_e8k3_bf16")
    r = oracle.moe_forward(c["x"], c["gate_w"], None, c["experts"], c["k"], c["tile"])
    T = c["x"].numel() // c["d"]
    for e, p in enumerate(r.perm):
        assert torch.equal(p, torch.sort(p).values)
        brute = [t for t in range(T) for j in range(c["k"])
                 if int(r.topi.reshape(T, -1)[t, j]) == e and float(r.topw.reshape(T, -1)[t, j]) > 0]
        assert p.tolist() == brute


def test_zero_weight_slot_is_not_dispatched(g):
    # k=3 picks an expert whose probability underflowed to 0: it is in topi
    # but has weight 0, so it is not counted or executed (model.py:576).
    c = load_moe_case(g, "moe_zero_weight")
    assert c["topi"].reshape(-1, 3)[0].tolist() == [0, 4, 6]
    assert c["counts"] == [4, 0, 0, 0, 4, 0, 0, 0]


# --------------------------------------------------------------------------
# linear attention (oracle/attn.c), pinned to the reference kernel
# --------------------------------------------------------------------------
GOLD_ATTN = os.path.join(os.path.dirname(__file__), "golden", "golden_attn.npz")


def _attn_inputs(B, T, H, D, seed):
    gen = torch.Generator().manual_seed(seed)
    Q = torch.nn.functional.elu(torch.randn(B, T, H, D, generator=gen)) + 1
    K = torch.nn.functional.elu(torch.randn(B, T, H, D, generator=gen)) + 1
    V = torch.randn(B, T, H, D, generator=gen)
    return Q, K, V


def _attn_golden_case(ga, i):
    def get(n):
        k = f"a{i}_{n}"
        return torch.from_numpy(ga[k]) if k in ga else None
    return {n: get(n) for n in ("Q", "K", "V", "Y", "DEN", "S", "z", "q", "k", "v", "y1", "S1", "z1")}


def test_attn_oracle_matches_golden():
    """Bit-exact against vectors written from the reference's attn_cpu.cpp."""
    ga = np.load(GOLD_ATTN)
    for i, eps in enumerate(ga["eps"].tolist()):
        c = _attn_golden_case(ga, i)
        Y, DEN, S, z = oracle.attn_forward(c["Q"], c["K"], c["V"], eps)
        assert torch.equal(Y, c["Y"]) and torch.equal(DEN, c["DEN"]) and torch.equal(z, c["z"]), i
        if c["S"] is not None:
            assert torch.equal(S, c["S"]), i
        y1, S1, z1 = oracle.attn_step(S, z, c["q"], c["k"], c["v"], eps)
        assert torch.equal(y1, c["y1"]) and torch.equal(z1, c["z1"]), i
        if c["S1"] is not None:
            assert torch.equal(S1, c["S1"]), i


@pytest.mark.skipif(oracle.ref_attn_module() is None, reason="oracle/_ref (reference attn_cpu.cpp) not built")
@pytest.mark.parametrize("B,T,H,D", [(2, 37, 3, 64), (1, 5, 2, 13), (2, 64, 4, 128), (1, 3, 1, 200),
                                     (1, 0, 2, 8), (1, 40, 1, 7)])
def test_attn_oracle_matches_reference_kernel(B, T, H, D):
    """Bit-exact against the reference's own attn_cpu.cpp (oracle/_ref), forward and step."""
    Q, K, V = _attn_inputs(B, T, H, D, B * 1000 + T * 10 + D)
    ref = oracle.ref_attn_module()
    Y, DEN, S, z = oracle.attn_forward(Q, K, V)
    Yr, Dr, Sr, zr = ref.attn_forward(Q, K, V, 1e-6, True, True)
    assert torch.equal(Y, Yr) and torch.equal(S, Sr) and torch.equal(z, zr)
    if T:
        assert torch.equal(DEN, Dr)
        q, k, v = Q[:, 0].contiguous(), K[:, 0].contiguous(), V[:, 0].contiguous()
        y1, S1, z1 = oracle.attn_step(S, z, q, k, v)
        S2, z2 = S.clone(), z.clone()
        y2, _, _ = ref.attn_step(S2, z2, q, k, v, 1e-6)
        assert torch.equal(y1, y2) and torch.equal(S1, S2) and torch.equal(z1, z2)


def test_attn_oracle_textbook_and_closed_forms():
    """Within fp32 rounding of the textbook recurrence (model.py:199-218), and a
    planted mistake -- z updated after den instead of before -- is not."""
    Q, K, V = _attn_inputs(2, 50, 3, 32, 5)
    Y = oracle.attn_forward(Q, K, V)[0]
    R = oracle.attn_textbook(Q, K, V)
    assert float(((Y - R).abs() / R.abs().clamp_min(1e-3)).max()) < 1e-4
    # planted: den from the state before this step's key
    B, T, H, D = Q.shape
    S = torch.zeros(B, H, D, D)
    z = torch.zeros(B, H, D)
    bad = []
    for t in range(T):
        kt = K[:, t] / K[:, t].norm(dim=-1, keepdim=True).clamp_min(1e-6)
        den = (Q[:, t] * z).sum(-1, keepdim=True).clamp_min(1e-6)
        S = S + kt.unsqueeze(-1) @ V[:, t].unsqueeze(-2)
        z = z + kt
        bad.append((Q[:, t].unsqueeze(-2) @ S).squeeze(-2) / den)
    assert float((torch.stack(bad, 1) - Y).abs().max()) > 1e-2
    # T=1 from zero state: y = v * (q.kn) / max(q.kn, eps) = v when q.kn >= eps
    Q1, K1, V1 = _attn_inputs(1, 1, 2, 16, 6)
    Y1 = oracle.attn_forward(Q1, K1, V1)[0]
    assert float((Y1 - V1).abs().max()) < 1e-5
    # all-zero keys: kn = 0 (the 1e-6 clamp), den clamps to eps, y = 0
    Yz, DENz, Sz, zz = oracle.attn_forward(Q1, torch.zeros_like(K1), V1)
    assert torch.equal(Yz, torch.zeros_like(Yz)) and float(DENz.max()) == np.float32(1e-6)
    assert torch.equal(Sz, torch.zeros_like(Sz))


@pytest.mark.skipif(oracle.ref_module() is None, reason="oracle/_ref (reference fp8_cpu.cpp) not built")
@pytest.mark.parametrize("rows,in_f,out_f,tile", [(64, 128, 128, 64), (33, 70, 100, 64), (16, 8, 64, 64),
                                                  (50, 300, 130, 32), (17, 96, 200, 128)])
def test_backward_input_bit_exact_with_reference_kernel(rows, in_f, out_f, tile):
    """The C restatement of fp8_backward_input (eight-way split fast path and
    the (g*lut)*s remainder) against the reference's own kernel, bit for bit,
    and against the decoded-weight product."""
    gen = torch.Generator().manual_seed(rows + in_f + out_f)
    g = torch.randn(rows, out_f, generator=gen)
    w, s = oracle.quantize_tiles(torch.randn(out_f, in_f, generator=gen) * 0.05, tile)
    dx = oracle.fp8_backward_input(g, w, s, in_f, out_f, tile)
    ref = oracle.ref_module().fp8_backward_input(g, w.reshape(-1).contiguous(), s.reshape(-1).contiguous(),
                                                 in_f, out_f, tile)
    assert torch.equal(dx, ref)
    bf = g.double() @ oracle.decode_full(w, s, tile).double()
    assert float((dx.double() - bf).abs().max() / bf.abs().max()) < 1e-5


def c1_layer_case(layer):
    """Layer `layer` of the config-1 model in golden_model_c1.npz: the exact
    bf16 input the reference Block handed to its SwiFFN_MoE, the layer's
    output, last_prob, top-k and counts, and the layer's weights (regenerated
    by tests/_model.draw_state, as the fixture's model was loaded)."""
    from _model import C1, draw_state
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_model_c1.npz"))
    sd, _ = draw_state(oracle.quantize_tiles)
    d, E = C1["d"], C1["experts"]
    p = f"blocks.{layer}.ffn."
    experts = [oracle.ExpertWeights(*[sd[p + f"experts.{e}.{n}.{t}"] for n in ("gate", "up", "down")
                                      for t in ("w8", "sc")]) for e in range(E)]
    x = torch.from_numpy(g[f"layer{layer}_moe_x"]).view(torch.bfloat16).reshape(-1, d)
    fx = torch.from_numpy(g[f"layer{layer}_moe_fx"]).view(torch.bfloat16).reshape(-1, d)
    prob = torch.from_numpy(g[f"layer{layer}_moe_prob"]).reshape(-1, E)
    topi = torch.from_numpy(g[f"layer{layer}_topi"]).reshape(-1, C1["top_k"])
    counts = g[f"layer{layer}_counts"].tolist()
    return x, sd[p + "gate.weight"], experts, fx, prob, topi, counts


@pytest.mark.parametrize("layer", [0, 1])
def test_moe_oracle_matches_reference_layer_in_model(layer):
    """The oracle's MoE layer (the C restatement of fp8_cpu.cpp in the
    model.py:557-585 loop) on the exact input the reference model's layer saw
    reproduces that layer's output, probabilities, top-k and counts bit for
    bit (golden_model_c1.npz, written by the reference SmaulLinear)."""
    from _model import C1
    x, gw, experts, fx, prob, topi, counts = c1_layer_case(layer)
    r = oracle.moe_forward(x, gw, None, experts, C1["top_k"], C1["tile"])
    assert torch.equal(r.topi, topi) and r.counts == counts
    assert torch.equal(r.prob, prob)
    assert torch.equal(r.out, fx)


@pytest.mark.skipif(oracle.ref_attn_module() is None, reason="oracle/_ref (reference attn_cpu.cpp) not built")
@pytest.mark.parametrize("B,T,H,D", [(2, 37, 3, 64), (1, 5, 2, 13), (1, 24, 2, 128), (1, 3, 1, 200),
                                     (1, 0, 2, 8), (1, 40, 1, 7), (1, 1, 1, 1)])
def test_attn_backward_oracle_matches_reference_kernel(B, T, H, D):
    """The backward (attn_cpu.cpp:227-368) bit-exact against the reference's own
    kernel (oracle/_ref), including the 8-lane sums of dq and dk and the
    scalar remainders (D = 13, 7, 1)."""
    Q, K, V = _attn_inputs(B, T, H, D, B * 977 + T * 13 + D)
    dY = torch.randn(B, T, H, D, generator=torch.Generator().manual_seed(D + T))
    Y, DEN, _, _ = oracle.attn_forward(Q, K, V)
    got = oracle.attn_backward(dY, Q, K, V, Y, DEN)
    ref = oracle.ref_attn_module().attn_backward(dY, Q, K, V, Y, DEN, 1e-6)
    for a, b in zip(got, ref):
        assert torch.equal(a, b)


def test_attn_backward_oracle_zero_keys_and_large_eps():
    """All-zero keys hit the 1e-6 clamp of the key norm (and its guarded
    nc^3 division); a large eps clamps every den.  Bit-exact with the
    reference kernel where it is built, finite always."""
    Q, K, V = _attn_inputs(1, 9, 2, 16, 3)
    K[:, 2:5] = 0.0
    dY = torch.randn(1, 9, 2, 16, generator=torch.Generator().manual_seed(4))
    for eps in (1e-6, 50.0):
        Y, DEN, _, _ = oracle.attn_forward(Q, K, V, eps)
        got = oracle.attn_backward(dY, Q, K, V, Y, DEN, eps)
        assert all(torch.isfinite(g).all() for g in got)
        ref = oracle.ref_attn_module()
        if ref is not None:
            for a, b in zip(got, ref.attn_backward(dY, Q, K, V, Y, DEN, eps)):
                assert torch.equal(a, b)


def test_attn_backward_oracle_vs_autograd_and_planted_mistake():
    """Within fp32 rounding of autograd (float64) through the textbook
    recurrence (model.py:199-233); a planted mistake -- the key norm treated
    as a constant, dropping the normalisation's backward term from dK -- is
    not."""
    Q, K, V = _attn_inputs(2, 30, 2, 24, 8)
    dY = torch.randn(2, 30, 2, 24, generator=torch.Generator().manual_seed(9))
    Y, DEN, _, _ = oracle.attn_forward(Q, K, V)
    dQ, dK, dV = oracle.attn_backward(dY, Q, K, V, Y, DEN)

    def grads(detach_norm):
        q, k, v = (t.double().requires_grad_(True) for t in (Q, K, V))
        B, T, H, D = q.shape
        S = torch.zeros(B, H, D, D, dtype=torch.float64)
        z = torch.zeros(B, H, D, dtype=torch.float64)
        ys = []
        for t in range(T):
            kt = k[:, t]
            nrm = kt.norm(dim=-1, keepdim=True).clamp_min(1e-6)
            kt = kt / (nrm.detach() if detach_norm else nrm)
            S = S + kt.unsqueeze(-1) @ v[:, t].unsqueeze(-2)
            z = z + kt
            num = (q[:, t].unsqueeze(-2) @ S).squeeze(-2)
            den = (q[:, t] * z).sum(-1, keepdim=True).clamp_min(1e-6)
            ys.append(num / den)
        torch.stack(ys, 1).backward(dY.double())
        return q.grad, k.grad, v.grad

    def rel(a, b):
        return float((a.double() - b).abs().max() / b.abs().max())
    ref = grads(False)
    for a, b in zip((dQ, dK, dV), ref):
        assert rel(a, b) < 1e-4
    planted = grads(True)
    assert rel(dK, planted[1]) > 1e-2
