"""Test harness: the SmaulLinear trunk (model.py:608-810) composed from this package.

TEST INFRASTRUCTURE.  The product here is the backend and its modules; the
model around them (embedding, RMSNorms, Block, LM head) is out of its scope.
This harness restates just enough of model.py's eval-mode trunk to run the
reference's whole forward / prefill / step on the GPU through the rocm
backend -- FP8Linear for every projection, ``attn_forward`` / ``attn_step``
for the linear-attention core and SwiFFN_MoE for the FFN -- so the result can
be compared with the reference model's own outputs (tests/golden/
golden_model_c1.npz, written by make_golden_model.py).

The weights are not stored: ``draw_state`` regenerates them from a seed in a
fixed order, keyed by the reference's state_dict names, and the fixture
generator loads the same dict into the reference model with strict=True.
"""
import torch
import torch.nn.functional as F

# Config 1 at 2 layers: d=512, 8 heads (D=64),
# ffn_mult 2.5 (h=1280), 4 SwiGLU experts top-2, tile 64, byte vocab 256.
C1 = dict(vocab=256, d=512, layers=2, heads=8, ffn_mult=2.5, experts=4, top_k=2, tile=64, eps=1e-6,
          batch=2, ctx=256, seed=1234)
NORMS = ("n1", "n2", "n3", "n4", "n5")
PROJ = ("q", "k", "v", "o")
EXPERT_PROJ = ("gate", "up", "down")


def draw_state(quantize, cfg=C1):
    """(state dict keyed like SmaulLinear.state_dict(), idx [B, ctx]).

    One CPU generator seeded cfg['seed'], draws in this order: idx
    U{0..vocab-1}; embedding N(0,0.02); n0 1+0.1*N(0,1); per layer the five
    norms (1+0.1*N), q/k/v/o N(0,0.02) quantized, the router N(0,0.02), and
    per expert gate/up/down N(0,0.02) quantized; nf; head N(0,0.02).
    ``quantize(w32, tile) -> (codes, scales)`` is the tiled-E4M3 quantizer.
    """
    d, V, E, tile = cfg["d"], cfg["vocab"], cfg["experts"], cfg["tile"]
    h = int(d * cfg["ffn_mult"])
    gen = torch.Generator().manual_seed(cfg["seed"])
    idx = torch.randint(0, V, (cfg["batch"], cfg["ctx"]), generator=gen)
    sd = {}

    def norm_w():
        return 1.0 + 0.1 * torch.randn(d, generator=gen)

    def fp8(prefix, o, i):
        w8, sc = quantize(torch.randn(o, i, generator=gen) * 0.02, tile)
        sd[prefix + ".w8"] = w8
        sd[prefix + ".sc"] = sc

    sd["emb.emb.weight"] = torch.randn(V, d, generator=gen) * 0.02
    sd["n0.weight"] = norm_w()
    for l in range(cfg["layers"]):
        p = f"blocks.{l}."
        for n in NORMS:
            sd[p + n + ".weight"] = norm_w()
        for q in PROJ:
            fp8(p + "att." + q, d, d)
        sd[p + "ffn.gate.weight"] = torch.randn(E, d, generator=gen) * 0.02
        for e in range(E):
            fp8(p + f"ffn.experts.{e}.gate", h, d)
            fp8(p + f"ffn.experts.{e}.up", h, d)
            fp8(p + f"ffn.experts.{e}.down", d, h)
    sd["nf.weight"] = norm_w()
    sd["head.weight"] = torch.randn(V, d, generator=gen) * 0.02
    return sd, idx


def rms(x, w, eps):
    """RMSNorm.forward (model.py:131-139)."""
    xf = x.float()
    v = xf.pow(2).mean(-1, keepdim=True)
    return (xf * torch.rsqrt(v + eps) * w).to(x.dtype if x.is_floating_point() else torch.float32)


class Trunk:
    """Eval-mode SmaulLinear (plain, fp8, MoE) on the rocm backend."""

    def __init__(self, sd, device, cfg=C1):
        from smaulnative_amd import FP8Linear, MoEConfig, SwiFFN_MoE
        from smaulnative_amd.compute import get_backend
        self.cfg, self.dev, self.be = cfg, device, get_backend("rocm")
        d, E = cfg["d"], cfg["experts"]
        self.H = cfg["heads"]
        self.D = d // self.H
        t = {k: v.to(device) for k, v in sd.items()}
        self.t = t

        def lin(prefix, i, o):
            m = FP8Linear(i, o, cfg["tile"]).to(device)
            m.w8.copy_(t[prefix + ".w8"])
            m.sc.copy_(t[prefix + ".sc"])
            return m

        self.layers = []
        for l in range(cfg["layers"]):
            p = f"blocks.{l}."
            att = {q: lin(p + "att." + q, d, d) for q in PROJ}
            moe = SwiFFN_MoE(MoEConfig(d_model=d, ffn_mult=cfg["ffn_mult"], tile=cfg["tile"], num_experts=E,
                                       num_experts_per_tok=cfg["top_k"])).to(device).eval()
            with torch.no_grad():
                moe.gate.weight.copy_(t[p + "ffn.gate.weight"])
                for e, ex in enumerate(moe.experts):
                    for nm in EXPERT_PROJ:
                        m = getattr(ex, nm)
                        m.w8.copy_(t[p + f"ffn.experts.{e}.{nm}.w8"])
                        m.sc.copy_(t[p + f"ffn.experts.{e}.{nm}.sc"])
            self.layers.append((att, moe, [t[p + n + ".weight"] for n in NORMS]))

    def _qkv(self, att, x, B, T):
        # LinearAttention._qkv (model.py:166-171): elu+1 features on q and k
        q = F.elu(att["q"](x).float().view(B, T, self.H, self.D)) + 1.0
        k = F.elu(att["k"](x).float().view(B, T, self.H, self.D)) + 1.0
        v = att["v"](x).float().view(B, T, self.H, self.D)
        return q, k, v

    def _tail(self, x, ax, moe, nw):
        # Block._tail (model.py:643-649)
        eps = self.cfg["eps"]
        a = rms(ax.float(), nw[1], eps)
        x = rms((x.float() + a.float()).to(x.dtype), nw[2], eps)
        fx = moe(x)
        f = rms(fx.float(), nw[3], eps)
        return rms((x.float() + f.float()).to(x.dtype), nw[4], eps)

    def _embed(self, idx):
        x = self.t["emb.emb.weight"][idx.to(self.dev)].to(torch.bfloat16)
        return rms(x.float(), self.t["n0.weight"], self.cfg["eps"]).to(torch.bfloat16)

    def _head(self, x):
        x = rms(x.float(), self.t["nf.weight"], self.cfg["eps"])
        return x.float() @ self.t["head.weight"].t()

    @torch.no_grad()
    def forward(self, idx):
        """SmaulLinear.forward (model.py:726-748): logits [B, T, V] and each layer's MoE top-k."""
        x = self._embed(idx)
        B, T, _ = x.shape
        eps = self.cfg["eps"]
        topi = []
        for att, moe, nw in self.layers:
            n1x = rms(x, nw[0], eps)
            q, k, v = self._qkv(att, n1x, B, T)
            y = self.be.attn_forward(q, k, v, eps, False)[0].reshape(B, T, -1)
            ax = att["o"](y.to(x.dtype))
            x = self._tail(x, ax, moe, nw)
            topi.append(moe.last_topi)
        return self._head(x), topi

    @torch.no_grad()
    def prefill(self, idx):
        """SmaulLinear.prefill (model.py:774-786): last-position logits and the attention states."""
        x = self._embed(idx)
        B, T, _ = x.shape
        eps = self.cfg["eps"]
        states = []
        for att, moe, nw in self.layers:
            n1x = rms(x, nw[0], eps)
            q, k, v = self._qkv(att, n1x, B, T)
            y, _, S, z = self.be.attn_forward(q, k, v, eps, False, need_state=True)
            ax = att["o"](y.reshape(B, T, -1).to(x.dtype))
            x = self._tail(x, ax, moe, nw)
            states.append((S, z))
        return self._head(x[:, -1:, :]), states

    @torch.no_grad()
    def step(self, idx, states):
        """SmaulLinear.step (model.py:788-810) for one token per sequence."""
        x = self._embed(idx)
        B = x.shape[0]
        eps = self.cfg["eps"]
        for i, (att, moe, nw) in enumerate(self.layers):
            n1x = rms(x, nw[0], eps)
            q, k, v = self._qkv(att, n1x, B, 1)
            S, z = states[i]
            y, S, z = self.be.attn_step(S, z, q[:, 0], k[:, 0], v[:, 0], eps)
            states[i] = (S, z)
            ax = att["o"](y.reshape(B, 1, -1).to(x.dtype))
            x = self._tail(x, ax, moe, nw)
        return self._head(x), states

