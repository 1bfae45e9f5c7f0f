"""Writes tests/golden/golden_model_c1.npz: the reference SmaulLinear's own outputs at a C1 shape.

    python tests/golden/make_golden_model.py

Run in the build container only (the reference is not present on the GPU box).
The model is config 1 cut to 2 layers: d=512, 8
heads, ffn_mult 2.5, 4 SwiGLU experts top-2, tile 64, byte vocab, batch 2 x
ctx 256.  Its weights come from tests/_model.draw_state (a seeded recipe keyed
by the reference's state_dict names, loaded with strict=True); the GEMM and
the attention recurrence are the reference's own kernel/fp8_cpu.cpp and
kernel/attn_cpu.cpp, compiled from source under oracle/_ref (their JIT loader
is never run); the quantizer is the reference's torch path.

Stored: idx, logits of forward (model.py:726-748) at five positions, each
layer's MoE top-k and expert counts, and the logits of prefill over the
first 255 tokens (model.py:774-786) followed by one step (model.py:788-810).
For each layer's SwiFFN_MoE in that forward, also its exact input (the bf16
x that Block hands to self.ffn, model.py:646), its output fx and its
last_prob, so the MoE layer can be checked on the reference's own inputs
(bf16 stored as int16 bit patterns).  The GPU test regenerates the weights
from the same recipe.

Also stored, as the scale for the GPU test's tolerance: how far the same
reference model moves when only the fp32 summation order of its fp8 GEMM
changes (the decoded weight through torch's CPU matmul instead of the native
kernel) -- the logits' rel-L2 at the five positions and the per-layer routing
agreement.  A bf16 trunk turns such reorderings into bf16 rounding flips and
occasional routing flips, so no reordered implementation can be closer.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REF = os.environ.get("SMAUL_REFERENCE", "/root/reference")
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "tests"))
sys.path.insert(0, REF)

import oracle  # noqa: E402  (only for oracle/_ref, the reference kernel builds)
from _model import C1, draw_state  # noqa: E402
from kernel import compute as ref_compute  # noqa: E402
from kernel import fp8_tile as ref_fp8  # noqa: E402
import model as ref_model  # noqa: E402

POSITIONS = [0, 1, 63, 128, 255]


def main():
    be = ref_compute.get_backend("cpu")
    fp8_mod, attn_mod = oracle.ref_module(), oracle.ref_attn_module()
    if fp8_mod is None or attn_mod is None:
        raise SystemExit("build oracle/_ref first: make -C oracle")
    be._ext = fp8_mod
    be._attn = attn_mod
    be._quant = False
    cfg = ref_model.LinearConfig(vocab_size=C1["vocab"], d_model=C1["d"], n_layer=C1["layers"],
                                 n_heads=C1["heads"], ffn_mult=C1["ffn_mult"], eps=C1["eps"], tile=C1["tile"],
                                 is_moe=True, num_experts=C1["experts"], num_experts_per_tok=C1["top_k"],
                                 precision="fp8", architecture="plain")
    torch.manual_seed(0)
    m = ref_model.SmaulLinear(cfg).eval()
    sd, idx = draw_state(ref_fp8.quantize_tiles)
    m.load_state_dict(sd, strict=True)
    out = {"idx": idx.numpy(), "positions": np.array(POSITIONS, dtype=np.int64)}
    seen = {}

    def capture(l):
        def hook(mod, inp, res):
            if l not in seen:  # the first forward only
                seen[l] = True
                assert inp[0].dtype == torch.bfloat16 and res.dtype == torch.bfloat16
                out[f"layer{l}_moe_x"] = inp[0].detach().contiguous().view(torch.int16).numpy()
                out[f"layer{l}_moe_fx"] = res.detach().contiguous().view(torch.int16).numpy()
                out[f"layer{l}_moe_prob"] = mod.last_prob.detach().float().numpy()
        return hook
    hooks = [blk.ffn.register_forward_hook(capture(l)) for l, blk in enumerate(m.blocks)]
    with torch.no_grad():
        logits, _ = m(idx)
        out["forward_logits"] = logits[:, POSITIONS, :].numpy()
        for l, blk in enumerate(m.blocks):
            out[f"layer{l}_topi"] = blk.ffn.last_topi.numpy()
            out[f"layer{l}_counts"] = np.array(blk.ffn.expert_token_counts, dtype=np.int64)
    for hk in hooks:
        hk.remove()
    pl, states = m.prefill(idx[:, :-1])
    sl, _ = m.step(idx[:, -1:], states)
    out["prefill_logits"] = pl.numpy()
    out["step_logits"] = sl.numpy()
    # the noise floor: the same model with the fp8 GEMM summed in another order
    native = be.fp8_forward

    def reordered(x, w, s, in_f, out_f, tile):
        W = oracle.decode_full(w.reshape(out_f, in_f), s.reshape(out_f, -1), tile)
        return x.float() @ W.T

    be.fp8_forward = reordered
    with torch.no_grad():
        alt, _ = m(idx)
        agree = [float((blk.ffn.last_topi == torch.from_numpy(out[f"layer{l}_topi"])).all(-1).float().mean())
                 for l, blk in enumerate(m.blocks)]
    be.fp8_forward = native
    a, r = alt[:, POSITIONS].double(), logits[:, POSITIONS].double()
    out["reorder_rel_l2"] = np.array(float((a - r).norm() / r.norm()))
    out["reorder_routing_agreement"] = np.array(agree)
    print("reordered GEMM: rel-L2", float(out["reorder_rel_l2"]), "routing agreement", agree)
    path = os.path.join(HERE, "golden_model_c1.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")
    print("forward vs prefill+step at the last position, max abs diff:",
          float((logits[:, -1] - sl[:, 0]).abs().max()))


if __name__ == "__main__":
    main()
