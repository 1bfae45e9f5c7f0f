"""The checkpoint loader (smaulnative_amd.loader): key layout, strictness, dtype restore.

CPU tests build small checkpoints in the reference's format (config.json +
model.safetensors with the merge_moe.py:110-119 expert keys) and load them
to the host; the GPU tests load to the device and run the layer."""
import json
import os

import pytest
import torch
from safetensors.torch import save_file

import oracle
from smaulnative_amd.loader import load_into, load_moe_layers, read_config

CFG = dict(vocab_size=256, d_model=128, n_layer=2, n_heads=2, ffn_mult=2.5, eps=1e-6, tile=64, is_moe=True,
           num_experts=4, num_experts_per_tok=2, precision="fp8", architecture="plain")


def write_ckpt(path, cfg=CFG, sc_dtype=torch.float32, seed=0, drop=None, extra=None, reshape=None):
    """A checkpoint with the MoE tensors of cfg (plus a non-MoE tensor, as a real one has)."""
    gen = torch.Generator().manual_seed(seed)
    d, E = cfg["d_model"], cfg["num_experts"]
    h = int(d * cfg["ffn_mult"])
    sd = {"emb.emb.weight": torch.randn(cfg["vocab_size"], d, generator=gen)}
    for l in range(cfg["n_layer"]):
        sd[f"blocks.{l}.ffn.gate.weight"] = torch.randn(E, d, generator=gen) * 0.02
        for e in range(E):
            for p, (o, i) in (("gate", (h, d)), ("up", (h, d)), ("down", (d, h))):
                w8, sc = oracle.quantize_tiles(torch.randn(o, i, generator=gen) * 0.02, cfg["tile"])
                sd[f"blocks.{l}.ffn.experts.{e}.{p}.w8"] = w8
                sd[f"blocks.{l}.ffn.experts.{e}.{p}.sc"] = sc.to(sc_dtype)
    if drop:
        del sd[drop]
    if extra:
        sd[extra] = torch.zeros(4)
    if reshape:
        sd[reshape] = sd[reshape][:-1].contiguous()
    os.makedirs(path, exist_ok=True)
    save_file(sd, os.path.join(path, "model.safetensors"))
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)
    return sd


def test_loads_every_moe_tensor_in_the_merge_layout(tmp_path):
    sd = write_ckpt(tmp_path)
    layers = load_moe_layers(tmp_path, device="cpu", prepare=False)
    assert [l.index for l in layers] == [0, 1] and layers[0].top_k == 2 and layers[0].tile == 64
    for l in layers:
        assert torch.equal(l.gate_weight, sd[f"blocks.{l.index}.ffn.gate.weight"]) and l.gate_bias is None
        for e, bufs in enumerate(l.experts):
            want = [sd[f"blocks.{l.index}.ffn.experts.{e}.{p}.{b}"] for p in ("gate", "up", "down")
                    for b in ("w8", "sc")]
            assert all(torch.equal(a, b) and a.dtype == b.dtype for a, b in zip(bufs, want))
    one = load_moe_layers(tmp_path, device="cpu", layers=[1], prepare=False)
    assert [l.index for l in one] == [1]


def test_bf16_scales_restored_to_fp32(tmp_path):
    sd = write_ckpt(tmp_path, sc_dtype=torch.bfloat16)
    l0 = load_moe_layers(tmp_path, device="cpu", prepare=False)[0]
    sc = l0.experts[0][1]
    assert sc.dtype == torch.float32
    assert torch.equal(sc, sd["blocks.0.ffn.experts.0.gate.sc"].float())


@pytest.mark.parametrize("kind", ["drop", "extra", "reshape", "not_moe"])
def test_strict_keys_and_shapes(tmp_path, kind):
    if kind == "drop":
        write_ckpt(tmp_path, drop="blocks.1.ffn.experts.3.down.sc")
        err = "missing"
    elif kind == "extra":
        write_ckpt(tmp_path, extra="blocks.0.ffn.experts.4.gate.w8")
        err = "unexpected"
    elif kind == "reshape":
        write_ckpt(tmp_path, reshape="blocks.0.ffn.experts.1.up.w8")
        err = "shape"
    else:
        write_ckpt(tmp_path, cfg=dict(CFG, is_moe=False))
        with pytest.raises(ValueError, match="not a MoE"):
            read_config(tmp_path)
        return
    with pytest.raises(RuntimeError, match=err):
        load_moe_layers(tmp_path, device="cpu", prepare=False)


@pytest.mark.gpu
def test_loaded_layer_runs_and_tracks_rewrites(tmp_path):
    """On the device: the loaded layer's forward equals the module's on the
    same buffers; 0x7F/0xFF codes (= +-448, like 0x7E/0xFE) stay stored as
    they are and give the same output; an in-place rewrite of w8 (what requant
    does, kernel/fp8_tile.py:252-253) is picked up by the repack cache."""
    from smaulnative_amd import MoEConfig, SwiFFN_MoE
    sd = write_ckpt(tmp_path, sc_dtype=torch.bfloat16)
    # plant 0x7F / 0xFF where the quantizer chose 0x7E / 0xFE
    k = "blocks.0.ffn.experts.1.up.w8"
    w = sd[k].clone()
    w[w == 0x7E] = 0x7F
    w[w == 0xFE] = 0xFF
    assert int((w == 0x7F).sum()) > 0
    sd_planted = dict(sd)
    sd_planted[k] = w
    save_file(sd_planted, os.path.join(tmp_path, "model.safetensors"))
    layers = load_moe_layers(tmp_path, device="cuda")
    l0 = layers[0]
    assert torch.equal(l0.experts[1][2].cpu(), w)          # stored codes unchanged
    x = torch.randn(300, CFG["d_model"]).to(torch.bfloat16).cuda()
    out, prob, topi, counts = l0.forward(x)
    moe = SwiFFN_MoE(MoEConfig(d_model=CFG["d_model"], ffn_mult=CFG["ffn_mult"], num_experts=4,
                               num_experts_per_tok=2)).cuda().eval()
    load_into(moe, l0)
    with torch.no_grad():
        ref = moe(x)
    assert torch.equal(out, ref)
    experts = [oracle.ExpertWeights(*[t.cpu() for t in ex]) for ex in l0.experts]
    r = oracle.moe_forward(x.cpu(), l0.gate_weight.cpu(), None, experts, 2)
    assert torch.equal(topi.cpu(), r.topi)
    assert float((out.cpu().double() - r.out.double()).norm() / r.out.double().norm()) < 2e-3
    # rewrite every expert's codes in place: the next forward follows them
    with torch.no_grad():
        for ex in l0.experts:
            for code in (ex[0], ex[2], ex[4]):
                code.copy_(torch.flip(code, dims=[1]))
    out2 = l0.forward(x)[0]
    experts2 = [oracle.ExpertWeights(*[t.cpu() for t in ex]) for ex in l0.experts]
    r2 = oracle.moe_forward(x.cpu(), l0.gate_weight.cpu(), None, experts2, 2)
    assert float((out2.cpu().double() - r2.out.double()).norm() / r2.out.double().norm()) < 2e-3
    assert not torch.equal(out2, out)
