"""Seeded synthetic inputs for the five benchmark/parity configurations of the MXFP8 SwiGLU-MLP path.

Every tensor is drawn on the CPU from its own ``torch.Generator`` (seed = 1000 * config + 100 * layer + index)
in fp32 and rounded to bf16 (RNE) where the path takes bf16, so the same bits can be copied to the GPU.
LoRA A/B stay fp32, as PEFT keeps them (the path casts them to bf16 once per step).

Config 5 ("outliers") draws x and dy from a Student-t(3) with NumPy's PCG64, scales 0.1% of the channels by
100 and injects blocks that exercise the E8M0 scale choice, the +-448 saturation boundary and E4M3 RNE ties.

"N(0, 1e-2)" for the upstream gradient is read as standard deviation 1e-2.
"""
import numpy as np
import torch

CONFIGS = {
    1: dict(name="c1", T=256, K=1024, N=3584, r=16, alpha=32, backward=False, layers=1),
    2: dict(name="c2", T=4096, K=1024, N=3584, r=16, alpha=32, backward=True, layers=1),
    3: dict(name="c3", T=10752, K=2048, N=6144, r=16, alpha=32, backward=True, layers=1),
    4: dict(name="c4", T=142336, K=2048, N=6144, r=16, alpha=32, backward=True, layers=24),
    5: dict(name="c5", T=10752, K=2048, N=6144, r=16, alpha=32, backward=True, layers=1, outliers=True),
}
DESCRIPTIONS = {
    1: "MXFP8 SwiGLU MLP fwd, M=256 d_model=1024 d_ffn=3584, LoRA r16 a32",
    2: "Qwen3.5-0.8B-shaped MLP fwd+bwd, M=4096 d_model=1024 d_ffn=3584, LoRA r16 a32",
    3: "Qwen3.5-2B-shaped MLP fwd+bwd, M=10752 d_model=2048 d_ffn=6144, LoRA r16 a32",
    4: "24-layer stack of Qwen3.5-2B-shaped MLPs fwd+bwd, M=142336 (16x8896) d_model=2048 d_ffn=6144, LoRA r16",
    5: "outlier stress fwd+bwd, M=10752 d_model=2048 d_ffn=6144, Student-t(3) + injected MX edge blocks",
}
# tensor index in the seed table
_IDX = dict(x=0, Wg=1, Wu=2, Wd=3, Ag=4, Bg=5, Au=6, Bu=7, Ad=8, Bd=9, dy=10)


def seed_of(cfg, name, layer=0):
    return 1000 * cfg + 100 * layer + _IDX[name]


def _normal(shape, std, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32) * std


def flops(T, K, N, backward=True):
    """Algorithmic MX GEMM work: forward 6·T·K·N (gate|up 4TKN + down 2TKN), backward 6·T·K·N (dh 2TKN + dx
    4TKN).  The frozen base weights have no weight gradient; LoRA bf16 flops are not counted."""
    return (12 if backward else 6) * T * K * N


def quant_bytes(rows, cols, dual=False):
    """Algorithmic HBM bytes of one MX quantization of a bf16 [rows, cols] tensor: read 2 B, write a 1 B code
    and one scale byte per 32 elements (blocked tiles, padded rows included); the dual-axis variant writes
    codes and scales for both axes."""
    s = -(-rows // 128) * (cols // 128) * 512
    if not dual:
        return rows * cols * 3 + s
    st = -(-cols // 128) * (rows // 128) * 512
    return rows * cols * 4 + s + st


def quant_lora_bytes(T, K, rp, transposed=False):
    """Algorithmic HBM bytes of one quant_lora over x [T, K] bf16 with w [rp, K]: read x and w, write the MX codes
    and blocked scales of x and the bf16 product [T, rp] (with its zero-padded transpose [rp, ceil(T/128)*128])."""
    tpad = -(-T // 128) * 128
    return quant_bytes(T, K) + rp * K * 2 + T * rp * 2 + (rp * tpad * 2 if transposed else 0)


def lora_bwd_bytes(T, N, r, quant=True):
    """Algorithmic HBM bytes of one lora_bwd over dy [T, N] bf16: read dy, xa [T, r], B [N, r]; write d(xa) [T, r]
    bf16 and dB [N, r] fp32; with quantization also the codes and blocked scales of dy (the partial sums are
    implementation traffic, not counted)."""
    by = T * N * 2 + T * r * 2 * 2 + N * r * (2 + 4)
    return by + (quant_bytes(T, N) - T * N * 2 if quant else 0)


def res_lora_bytes(T, N, r):
    """Algorithmic HBM bytes of one res_lora: read x, y [T, N] and xa [T, r], B [N, r]; write out [T, N] (bf16)."""
    return T * N * 2 * 3 + (T + N) * r * 2


def _outlier_blocks(x, rng):
    """Inject MX edge cases into a bf16-valued fp32 [T, C] tensor in place (config 5)."""
    T, C = x.shape
    nb = C // 32
    # 0.1% of channels scaled x100 (round(0.001 * C) channels)
    nch = max(1, round(0.001 * C))
    ch = rng.choice(C, size=nch, replace=False)
    x[:, ch] *= 100.0
    rows = rng.permutation(T)
    k = 0

    def take(n):
        nonlocal k
        r = rows[k:k + n]
        k += n
        return r

    # all-zero blocks (+0.0) and -0.0 blocks
    for r in take(64):
        b = rng.integers(nb)
        x[r, 32 * b:32 * b + 32] = 0.0
    for r in take(16):
        b = rng.integers(nb)
        x[r, 32 * b:32 * b + 32] = -0.0
    # amax exactly +-448 * 2^k for k in [-20, 20]: the block max lands on the top code 0x7E / 0xFE
    for kk in range(-20, 21):
        for r in take(2):
            b = rng.integers(nb)
            blk = x[r, 32 * b:32 * b + 32]
            m = np.abs(blk).max()
            if m > 0:
                blk *= (224.0 * 2.0 ** kk) / m  # keep every other element below the boundary
            j = rng.integers(32)
            blk[j] = (448.0 if rng.random() < 0.5 else -448.0) * 2.0 ** kk
    # E4M3 RNE midpoints after scaling: amax 448·2^k fixes the scale to 2^k, then values m·2^k with m a tie
    ties = np.array([17.0, 19.0, 2.0 ** -10, 3 * 2.0 ** -10, 9.5, 10.5, 100.0, 116.0, 232.0, 432.0, 0.53125,
                     0.59375])
    for kk in (-6, 0, 3):
        for r in take(8):
            b = rng.integers(nb)
            blk = x[r, 32 * b:32 * b + 32]
            vals = rng.choice(ties, size=32) * np.where(rng.random(32) < 0.5, -1.0, 1.0)
            vals[0] = 448.0
            blk[:] = vals * 2.0 ** kk
    return x


def _student_t(shape, seed, scale=1.0):
    rng = np.random.Generator(np.random.PCG64(seed))
    x = rng.standard_t(3.0, size=shape).astype(np.float32) * scale
    return x, rng


def make_inputs(cfg, T=None, layer=0, dy=True, x=True):
    """CPU tensors for one layer of configuration ``cfg`` (1..5).  ``T`` overrides the token count (row
    subsets of the same shape).  Returns dict(x, Wg, Wu, Wd, Ag, Bg, Au, Bu, Ad, Bd, dy, s, T, K, N, r);
    ``x=False`` / ``dy=False`` leave out the activation / upstream gradient (layers > 0 of a stack)."""
    c = CONFIGS[cfg]
    T = c["T"] if T is None else T
    K, N, r = c["K"], c["N"], c["r"]
    s = c["alpha"] / r
    out = dict(T=T, K=K, N=N, r=r, s=s)
    if x:
        if c.get("outliers"):
            xf, rng = _student_t((T, K), seed_of(cfg, "x", layer))
            xf = torch.from_numpy(_outlier_blocks(xf, rng))
        else:
            xf = _normal((T, K), 1.0, seed_of(cfg, "x", layer))
        out["x"] = xf.to(torch.bfloat16)
    out["Wg"] = _normal((N, K), 0.02, seed_of(cfg, "Wg", layer)).to(torch.bfloat16)
    out["Wu"] = _normal((N, K), 0.02, seed_of(cfg, "Wu", layer)).to(torch.bfloat16)
    out["Wd"] = _normal((K, N), 0.02, seed_of(cfg, "Wd", layer)).to(torch.bfloat16)
    out["Ag"] = _normal((r, K), 0.02, seed_of(cfg, "Ag", layer))
    out["Bg"] = _normal((N, r), 0.02, seed_of(cfg, "Bg", layer))
    out["Au"] = _normal((r, K), 0.02, seed_of(cfg, "Au", layer))
    out["Bu"] = _normal((N, r), 0.02, seed_of(cfg, "Bu", layer))
    out["Ad"] = _normal((r, N), 0.02, seed_of(cfg, "Ad", layer))
    out["Bd"] = _normal((K, r), 0.02, seed_of(cfg, "Bd", layer))
    if dy:
        if c.get("outliers"):
            dyf, rng = _student_t((T, K), seed_of(cfg, "dy", layer), 1e-2)
            dyf = torch.from_numpy(_outlier_blocks(dyf, rng))
        else:
            dyf = _normal((T, K), 1e-2, seed_of(cfg, "dy", layer))
        out["dy"] = dyf.to(torch.bfloat16)
    return out


class LoraLinear(torch.nn.Module):
    """The attribute surface of a PEFT LoRA Linear that fused_linear._part reads (base_layer, lora_A/B
    ModuleDicts, scaling, active_adapters, lora_dropout, use_dora, merged, disable_adapters).  peft is not
    installed here; this stands in for it so the drop-in API can be driven as the training script drives it."""

    def __init__(self, base, A, B, alpha):
        super().__init__()
        r = A.shape[0]
        self.base_layer = base
        self.lora_A = torch.nn.ModuleDict({"default": torch.nn.Linear(A.shape[1], r, bias=False)})
        self.lora_B = torch.nn.ModuleDict({"default": torch.nn.Linear(r, B.shape[0], bias=False)})
        with torch.no_grad():
            self.lora_A["default"].weight.copy_(A)
            self.lora_B["default"].weight.copy_(B)
        self.lora_dropout = torch.nn.ModuleDict({"default": torch.nn.Identity()})
        self.scaling = {"default": alpha / r}
        self.active_adapters = ["default"]
        self.use_dora = {"default": False}
        self.merged = False
        self.disable_adapters = False

    def forward(self, x):
        a, b = self.lora_A["default"], self.lora_B["default"]
        return self.base_layer(x) + self.scaling["default"] * b(a(x))


class SwiGLUMLP(torch.nn.Module):
    """gate_proj / up_proj / down_proj with a SiLU act_fn, the shape of a Qwen3.5 MLP."""

    def __init__(self, inp, alpha):
        super().__init__()
        K, N = inp["K"], inp["N"]

        def lin(w):
            m = torch.nn.Linear(w.shape[1], w.shape[0], bias=False)
            with torch.no_grad():
                m.weight.copy_(w)
            m.weight.requires_grad_(False)
            return m

        self.gate_proj = LoraLinear(lin(inp["Wg"]), inp["Ag"], inp["Bg"], alpha)
        self.up_proj = LoraLinear(lin(inp["Wu"]), inp["Au"], inp["Bu"], alpha)
        self.down_proj = LoraLinear(lin(inp["Wd"]), inp["Ad"], inp["Bd"], alpha)
        self.act_fn = torch.nn.SiLU()

    def forward(self, x):
        return self.down_proj(self.act_fn(self.gate_proj(x)) * self.up_proj(x))


class _Layer(torch.nn.Module):
    def __init__(self, mlp):
        super().__init__()
        self.mlp = mlp


class _Decoder(torch.nn.Module):
    def __init__(self, mlps):
        super().__init__()
        self.layers = torch.nn.ModuleList([_Layer(m) for m in mlps])


class MLPStack(torch.nn.Module):
    """model.layers[i].mlp, named like a Hugging Face decoder ('model.layers.<i>.mlp.gate_proj...'): the module
    path mxfp8.enable_mxfp8 walks (names containing '.layers.')."""

    def __init__(self, mlps):
        super().__init__()
        self.model = _Decoder(mlps)

    @property
    def layers(self):
        return self.model.layers


class AttnProjections(torch.nn.Module):
    """q_proj / k_proj / v_proj / o_proj of an attention block as PEFT-shaped LoRA linears (frozen bf16 base
    weights N(0, 0.02), fp32 LoRA A/B N(0, 0.02)), the grouped MX linears of fused_linear.  Seeded from `seed`."""

    def __init__(self, K, nq, nkv, r, alpha, seed=0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)

        def lora(n_out, n_in):
            base = torch.nn.Linear(n_in, n_out, bias=False)
            with torch.no_grad():
                base.weight.copy_(torch.randn(n_out, n_in, generator=g) * 0.02)
            base.weight.requires_grad_(False)
            base.to(torch.bfloat16)
            return LoraLinear(base, torch.randn(r, n_in, generator=g) * 0.02, torch.randn(n_out, r, generator=g) * 0.02,
                              alpha)

        self.q_proj, self.k_proj, self.v_proj = lora(nq, K), lora(nkv, K), lora(nkv, K)
        self.o_proj = lora(K, nq)


def build_attn(K, nq, nkv, r, alpha, device="cuda", seed=0):
    """A one-layer decoder-shaped module ('model.layers.0.self_attn.q_proj...') holding AttnProjections, the path
    mxfp8.enable_mxfp8 walks."""
    m = torch.nn.Module()
    m.model = torch.nn.Module()
    layer = torch.nn.Module()
    layer.self_attn = AttnProjections(K, nq, nkv, r, alpha, seed)
    m.model.layers = torch.nn.ModuleList([layer])
    return m.to(device)


def build_model(cfg, T=None, layers=1, device="cuda"):
    """(model, inputs) for `layers` independent seeded layers of configuration cfg, bf16 frozen weights and
    fp32 LoRA parameters on `device`; inputs of layer 0 (x, dy) are returned on the CPU (the other layers'
    dicts hold their weights only: a stack feeds each layer the previous layer's output)."""
    c = CONFIGS[cfg]
    mlps, inps = [], []
    for layer in range(layers):
        inp = make_inputs(cfg, T=T, layer=layer, dy=(layer == 0), x=(layer == 0))
        m = SwiGLUMLP(inp, c["alpha"])
        for name in ("gate_proj", "up_proj", "down_proj"):
            getattr(m, name).base_layer.to(dtype=torch.bfloat16)
        mlps.append(m)
        inps.append(inp)
    model = MLPStack(mlps).to(device)
    return model, inps
