"""Pins of the MLP oracle (oracle/mlp.py) by what the mathematics fixes, on the CPU.

The GPU MLP tests compare the HIP path with oracle/mlp.py, so the oracle itself must be checked by something
that does not share its code.  The checks here use:

  * lossless MX inputs: activations whose 32-blocks are E4M3 values times a power of two, and weights on one
    power-of-two grid, so that MX quantization along either axis returns the input exactly.  The MX GEMMs of the
    path then equal exact products, and the only MX rounding left is that of h (forward) and of dg | du (dx);
  * an independent float64 composition of the forward (F.silu, F.linear-style float64 products, torch's own
    float8_e4m3fn cast for the h round trip) with the rounding points the reference names
    (/root/reference/scripts/fused_mlp.py:65-109, :263-293);
  * torch.autograd of the exact (unrounded) float64 MLP for every gradient of _MLP.backward
    (/root/reference/scripts/fused_mlp.py:112-175, :295-336), and float64 central differences of the same loss
    along random directions, which do not use autograd;
  * exact reductions: LoRA scalings 0 give the plain MX SwiGLU and exactly zero LoRA gradients; LoRA B = 0 gives
    exactly zero A gradients;
  * rounding-point pins: each bf16 tensor the reference rounds (dxa after its scaling, dB_d before and after its
    scaling, dx after the GEMM and after the addmm_) equals the bf16 rounding of the exact float64 value of its
    defining expression in the oracle's own preceding bf16 tensors;
  * mutants: the checks are run on copies of the oracle with one planted mistake each (gate/up swapped, dg/du
    swapped in the dx operand, s_d dropped from dB_d, dxa scaled after its bf16 rounding, a wrong SwiGLU
    derivative, the down LoRA-B product dropped, B_u in place of B_g, a permuted A_d, dB_d rounded once, the
    dx LoRA term dropped, W_gu in place of W_guᵀ), and the checks listed for each mutant in EXPECT must
    reject it.

LoRA scalings are deliberately not powers of two (1.5, 0.75, 1.25) so that scaling before or after a bf16
rounding gives different bits."""
import inspect
import types

import pytest
import torch
import torch.nn.functional as F

from oracle import mlp as omlp
from oracle import mx

F64, BF16 = torch.float64, torch.bfloat16
SCALES = (1.5, 0.75, 1.25)  # s_g, s_u, s_d


def _bf(t):
    return t.to(BF16).to(F64)


def _e4m3(t):
    """Nearest E4M3FN value (ties to even) of float64 values in [-448, 448], by torch's fp8 cast."""
    return t.clamp(-448, 448).to(torch.float32).to(torch.float8_e4m3fn).to(F64)


def _lossless(R, C, std, seed, per_block=True):
    """bf16 [R, C] whose 32-blocks along C are E4M3 values times a power of two (one per block, or one for the
    whole matrix so that the 32-blocks along R are too): MX quantization returns them exactly."""
    g = torch.Generator().manual_seed(seed)
    raw = torch.randn(R, C, generator=g, dtype=F64) * std
    if per_block:
        amax = raw.abs().view(R, C // 32, 32).amax(-1).clamp_min(1e-30)
        sc = torch.exp2(torch.ceil(torch.log2(amax / 448))).repeat_interleave(32, dim=1)
    else:
        sc = torch.full_like(raw, 2.0 ** float(torch.ceil(torch.log2(raw.abs().max() / 448))))
    return (_e4m3(raw / sc) * sc).to(BF16)


def _bf16_normal(shape, std, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * std).to(BF16)


def _mx_roundtrip(t):
    """Independent MX round trip along the last dim of float64 [R, C]: scale 2^ceil(log2(amax / 448)) per 32-block
    (1 for an all-zero block), codes by torch's RNE E4M3 cast."""
    R, C = t.shape
    b = t.reshape(R, C // 32, 32)
    amax = b.abs().amax(-1, keepdim=True)
    sc = torch.where(amax > 0, torch.exp2(torch.ceil(torch.log2(amax.clamp_min(1e-300) / 448))),
                     torch.ones_like(amax))
    return (_e4m3(b / sc) * sc).reshape(R, C)


def make_case(T=64, K=256, N=256, r=16, seed=0, scales=SCALES, zero_B=False):
    """Lossless MX inputs and bf16-valued LoRA weights (as the per-step casts of fused_mlp.py:272-276 give)."""
    s = 100 * seed
    c = dict(x=_lossless(T, K, 1.0, s + 1), dy=_lossless(T, K, 1e-2, s + 2),
             Wg=_lossless(N, K, 0.02, s + 3, per_block=False), Wu=_lossless(N, K, 0.02, s + 4, per_block=False),
             Wd=_lossless(K, N, 0.02, s + 5, per_block=False),
             Ag=_bf16_normal((r, K), 0.02, s + 6), Bg=_bf16_normal((N, r), 0.02, s + 7),
             Au=_bf16_normal((r, K), 0.02, s + 8), Bu=_bf16_normal((N, r), 0.02, s + 9),
             Ad=_bf16_normal((r, N), 0.02, s + 10), Bd=_bf16_normal((K, r), 0.02, s + 11))
    if zero_B:
        for k in ("Bg", "Bu", "Bd"):
            c[k] = torch.zeros_like(c[k])
    c["s"] = scales
    return c


def run_oracle(c, mod=omlp):
    W = mod.prepare_weights(c["Wg"], c["Wu"], c["Wd"])
    S, bg, bu, ad, bd = mod.lora_cast(c["Ag"], c["Bg"], c["Au"], c["Bu"], c["Ad"], c["Bd"])
    sg, su, sd = c["s"]
    f = mod.forward(c["x"], W, S, bg, bu, ad, bd, sg, su, sd)
    b = mod.backward(c["x"], f["xs"], f["gu"], W, S, bg, bu, ad, bd, sg, su, sd, c["dy"])
    return W, f, b


def compose_forward(c):
    """float64 restatement of the forward with the reference's bf16 rounding points; every MX GEMM operand but h
    is lossless, so its products are exact float64 products."""
    d = {k: v.to(F64) for k, v in c.items() if isinstance(v, torch.Tensor)}
    sg, su, sd = c["s"]
    r = d["Ag"].shape[0]
    xs = _bf(d["x"] @ torch.cat([d["Ag"], d["Au"]]).t())
    g = _bf(_bf(d["x"] @ d["Wg"].t()) + sg * (xs[:, :r] @ d["Bg"].t()))
    u = _bf(_bf(d["x"] @ d["Wu"].t()) + su * (xs[:, r:] @ d["Bu"].t()))
    h = _bf(F.silu(g) * u)
    xsd = _bf(h @ d["Ad"].t())
    y0 = _bf(_mx_roundtrip(h) @ d["Wd"].t())
    y = _bf(y0 + sd * (xsd @ d["Bd"].t()))
    return dict(xs=xs, g=g, u=u, h=h, xsd=xsd, y0=y0, y=y)


_GRADS = ("x", "Ag", "Bg", "Au", "Bu", "Ad", "Bd")
_ORACLE_GRAD = dict(x="dx", Ag="dA_g", Bg="dB_g", Au="dA_u", Bu="dB_u", Ad="dA_d", Bd="dB_d")


def exact_loss(p, c):
    """<y, dy> of the exact float64 MLP with LoRA (no rounding, no quantization), p = parameter dict."""
    sg, su, sd = c["s"]
    x = p["x"]
    g = x @ p["Wg"].t() + sg * (x @ p["Ag"].t()) @ p["Bg"].t()
    u = x @ p["Wu"].t() + su * (x @ p["Au"].t()) @ p["Bu"].t()
    h = F.silu(g) * u
    y = h @ p["Wd"].t() + sd * (h @ p["Ad"].t()) @ p["Bd"].t()
    return (y * p["dy"]).sum()


def exact_grads(c):
    p = {k: c[k].to(F64).requires_grad_(k in _GRADS) for k in ("x", "dy", "Wg", "Wu", "Wd") + _GRADS[1:]}
    gs = torch.autograd.grad(exact_loss(p, c), [p[k] for k in _GRADS])
    return dict(zip(_GRADS, gs))


def _rel(got, ref):
    got, ref = got.to(F64), ref.to(F64)
    return ((got - ref).abs().max() / ref.abs().max().clamp_min(1e-300)).item()


def _mismatch(got, ref):
    """Fraction of elements of two bf16-valued tensors that differ, and the largest difference in units of the
    bf16 spacing at the larger magnitude."""
    got, ref = got.to(F64), ref.to(F64)
    d = (got - ref).abs()
    mag = torch.maximum(got.abs(), ref.abs()).clamp_min(2.0 ** -126)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
    return (d > 0).double().mean().item(), (d / ulp).max().item()


# Bars.  The composition agrees with the oracle except where an fp32 (oracle) against float64 (composition) sum
# or exp lands on the other side of a bf16 rounding boundary: at most 1 ulp, in few elements.  Against the exact
# gradient the oracle carries the bf16 rounding of g, u, h, dh, dg, du, dxa, dxd and xS_down (a few 2^-9
# relative each); dx also carries the E4M3 rounding of dg | du (2^-4 relative per element at most).
FLIP_FRAC, FLIP_ULPS = 2e-3, 1.0
GRAD_TOL = dict(x=6e-2, Ag=1e-2, Bg=1e-2, Au=1e-2, Bu=1e-2, Ad=1e-2, Bd=1e-2)


# ------------------------------------------------------------------------------------------ the checks


def check_weights(c, mod=omlp):
    """prepare_weights (/root/reference/scripts/mxfp8.py:472-490): W_gu along K, W_guᵀ along 2N, W_down along N,
    W_downᵀ along K, each dequantizing to exactly the lossless weight."""
    W = mod.prepare_weights(c["Wg"], c["Wu"], c["Wd"])
    N, K = c["Wg"].shape
    Wgu = torch.cat([c["Wg"], c["Wu"]]).float()
    assert torch.equal(mx.dequant(W["w"], W["ws"], 2 * N, K), Wgu), "W_gu along K"
    assert torch.equal(mx.dequant(W["wt"], W["wts"], K, 2 * N), Wgu.t()), "W_gu^T along 2N"
    assert torch.equal(mx.dequant(W["dw"], W["dws"], K, N), c["Wd"].float()), "W_down along N"
    assert torch.equal(mx.dequant(W["dwt"], W["dwts"], N, K), c["Wd"].float().t()), "W_down^T along K"


def check_forward(c, mod=omlp):
    """Stage by stage on the oracle's own preceding bf16 tensors (a rounding flip upstream is not carried into
    the next stage, where cancellation in g = gu + LoRA would magnify it), then y end to end against the
    composition (/root/reference/scripts/fused_mlp.py:69-70, :104-109, :277-284)."""
    _, f, _ = run_oracle(c, mod)
    sg, su, sd = c["s"]
    d = {k: v.to(F64) for k, v in c.items() if isinstance(v, torch.Tensor)}
    o = {k: f[k].to(F64) for k in ("xs", "gu", "g", "u", "h", "xsd", "y0")}
    r, N = d["Ag"].shape[0], d["Wg"].shape[0]
    ref = dict(xs=_bf(d["x"] @ torch.cat([d["Ag"], d["Au"]]).t()),
               gu=_bf(d["x"] @ torch.cat([d["Wg"], d["Wu"]]).t()),
               g=_bf(o["gu"][:, :N] + sg * (o["xs"][:, :r] @ d["Bg"].t())),
               u=_bf(o["gu"][:, N:] + su * (o["xs"][:, r:] @ d["Bu"].t())),
               h=_bf(F.silu(o["g"]) * o["u"]),
               xsd=_bf(o["h"] @ d["Ad"].t()),
               y0=_bf(_mx_roundtrip(o["h"]) @ d["Wd"].t()),
               y=_bf(o["y0"] + sd * (o["xsd"] @ d["Bd"].t())))
    for k, v in ref.items():
        frac, ulps = _mismatch(f[k], v)
        assert frac <= FLIP_FRAC and ulps <= FLIP_ULPS, (k, frac, ulps)
    e = _rel(f["y"], compose_forward(c)["y"])
    assert e <= 1e-2, ("y end to end", e)


def check_autograd(c, mod=omlp):
    _, _, b = run_oracle(c, mod)
    ex = exact_grads(c)
    for k in _GRADS:
        e = _rel(b[_ORACLE_GRAD[k]], ex[k])
        assert e <= GRAD_TOL[k], (k, e)


def check_finite_differences(c, mod=omlp, n_dir=2, eps=1e-4):
    """<oracle gradient, v> against (L(p + eps v) - L(p - eps v)) / 2 eps of the exact float64 loss, with v the
    oracle gradient's own direction (a gradient uncorrelated with the true one gives a derivative near 0 there)
    and random unit directions (bar: tol * |gradient|, the Cauchy-Schwarz scale)."""
    _, _, b = run_oracle(c, mod)
    p = {k: c[k].to(F64) for k in ("x", "dy", "Wg", "Wu", "Wd") + _GRADS[1:]}
    gen = torch.Generator().manual_seed(7)
    for k in _GRADS:
        gk = b[_ORACLE_GRAD[k]].to(F64)
        norm = gk.norm().item()
        assert norm > 0, k
        dirs = [gk / norm] + [torch.randn(gk.shape, generator=gen, dtype=F64) for _ in range(n_dir)]
        for v in dirs:
            v = v / v.norm()
            pp, pm = dict(p), dict(p)
            pp[k], pm[k] = p[k] + eps * v, p[k] - eps * v
            fd = ((exact_loss(pp, c) - exact_loss(pm, c)) / (2 * eps)).item()
            got = (gk * v).sum().item()
            assert abs(got - fd) <= 2 * GRAD_TOL[k] * norm, (k, got, fd, norm)


def check_rounding_points(c, mod=omlp):
    """Each rounded tensor of the backward equals bf16(exact value of its defining expression) in the oracle's
    own preceding bf16 tensors (/root/reference/scripts/fused_mlp.py:155-159, :311-333)."""
    W, f, b = run_oracle(c, mod)
    sg, su, sd = c["s"]
    r = c["Ag"].shape[0]
    d = {k: c[k].to(F64) for k in ("x", "dy", "Wg", "Wu", "Wd", "Ag", "Au", "Bg", "Bu", "Ad", "Bd")}
    g, u, dh = b["g"].to(F64), b["u"].to(F64), b["dh"].to(F64)
    dg, du, h = b["dg"].to(F64), b["du"].to(F64), b["h"].to(F64)
    xs = f["xs"].to(F64)
    ref = {}
    ref["dxd"] = _bf(sd * _bf(d["dy"] @ d["Bd"]))                                   # :311-313
    ref["dhm"] = _bf(d["dy"] @ d["Wd"])                                              # :309, MX(dy) lossless
    ref["dh"] = _bf(b["dhm"].to(F64) + b["dxd"].to(F64) @ d["Ad"])                 # :155
    ref["du"] = _bf(dh * F.silu(g))                                                  # :157
    sig = torch.sigmoid(g)
    ref["dg"] = _bf(dh * u * sig * (1 + g * (1 - sig)))                              # :158-159
    ref["dxa"] = _bf(torch.cat([sg * (dg @ d["Bg"]), su * (du @ d["Bu"])], 1))      # :166-167, :319-326
    ref["dB_d"] = _bf(sd * _bf(d["dy"].t() @ _bf(h @ d["Ad"].t())))                 # :316-318
    ref["dA"] = _bf(b["dxa"].to(F64).t() @ d["x"])                                   # :333
    dgu = _mx_roundtrip(torch.cat([dg, du], 1))                                      # :160-162
    ref["dx0"] = _bf(dgu @ torch.cat([d["Wg"], d["Wu"]]))                            # :329
    ref["dx"] = _bf(b["dx0"].to(F64) + b["dxa"].to(F64) @ torch.cat([d["Ag"], d["Au"]]))  # :331
    for k, v in ref.items():
        frac, ulps = _mismatch(b[k], v)
        assert frac <= FLIP_FRAC and ulps <= FLIP_ULPS, (k, frac, ulps)
    # fp32 results the reference keeps unrounded: dB_g, dB_u (scaled), dA_d
    assert _rel(b["dB_g"], sg * (dg.t() @ xs[:, :r])) <= 1e-5
    assert _rel(b["dB_u"], su * (du.t() @ xs[:, r:])) <= 1e-5
    assert _rel(b["dA_d"], (h.t() @ b["dxd"].to(F64)).t()) <= 1e-5


def check_zero_scalings(c, mod=omlp):
    """s_g = s_u = s_d = 0: y is the plain MX SwiGLU of the frozen weights and every LoRA gradient is exactly 0."""
    c = dict(c, s=(0.0, 0.0, 0.0))
    _, f, b = run_oracle(c, mod)
    d = {k: c[k].to(F64) for k in ("x", "Wg", "Wu", "Wd")}
    h = _bf(F.silu(_bf(d["x"] @ d["Wg"].t())) * _bf(d["x"] @ d["Wu"].t()))
    frac, ulps = _mismatch(f["y"], _bf(_mx_roundtrip(h) @ d["Wd"].t()))
    assert frac <= FLIP_FRAC and ulps <= FLIP_ULPS, ("y", frac, ulps)
    for k in ("dA_g", "dA_u", "dA_d", "dB_g", "dB_u", "dB_d"):
        assert torch.count_nonzero(b[k]) == 0, k


def check_zero_B(c, mod=omlp):
    """LoRA B = 0 on all three projections: dA_g = dA_u = dA_d = 0 exactly, y is the plain MX SwiGLU."""
    c = dict(c)
    for k in ("Bg", "Bu", "Bd"):
        c[k] = torch.zeros_like(c[k])
    _, f, b = run_oracle(c, mod)
    for k in ("dA_g", "dA_u", "dA_d"):
        assert torch.count_nonzero(b[k]) == 0, k
    d = {k: c[k].to(F64) for k in ("x", "Wg", "Wu", "Wd")}
    h = _bf(F.silu(_bf(d["x"] @ d["Wg"].t())) * _bf(d["x"] @ d["Wu"].t()))
    frac, ulps = _mismatch(f["y"], _bf(_mx_roundtrip(h) @ d["Wd"].t()))
    assert frac <= FLIP_FRAC and ulps <= FLIP_ULPS, ("y", frac, ulps)


CHECKS = [check_weights, check_forward, check_autograd, check_finite_differences, check_rounding_points,
          check_zero_scalings, check_zero_B]


# ------------------------------------------------------------------------------------------ the oracle passes


@pytest.fixture(scope="module")
def case():
    return make_case()


@pytest.mark.parametrize("check", CHECKS, ids=lambda f: f.__name__)
def test_oracle_passes(check, case):
    check(case)


def test_oracle_passes_small_fd():
    """Central differences at T = 8 tokens and the smallest shapes the blocked layout takes."""
    check_finite_differences(make_case(T=8, K=128, N=128, seed=3), n_dir=3)


def test_oracle_passes_rank32_power_of_two_scalings():
    c = make_case(T=32, K=128, N=256, r=32, seed=5, scales=(2.0, 2.0, 2.0))
    for chk in (check_forward, check_autograd, check_rounding_points):
        chk(c)


def test_lossless_inputs_are_lossless(case):
    for k in ("x", "dy"):
        q, s = mx.quant(case[k])
        assert torch.equal(mx.dequant(q, s, *case[k].shape), case[k].float()), k


def test_need_out_false_saves_the_same(case):
    W = omlp.prepare_weights(case["Wg"], case["Wu"], case["Wd"])
    S, bg, bu, ad, bd = omlp.lora_cast(case["Ag"], case["Bg"], case["Au"], case["Bu"], case["Ad"], case["Bd"])
    a = omlp.forward(case["x"], W, S, bg, bu, ad, bd, *case["s"])
    z = omlp.forward(case["x"], W, S, bg, bu, ad, bd, *case["s"], need_out=False)
    assert torch.equal(a["xs"], z["xs"]) and torch.equal(a["gu"], z["gu"]) and "y" not in z


# ------------------------------------------------------------------------------------------ mutants


def _mutant(old, new):
    """A copy of oracle/mlp.py with one textual change (which must occur exactly once)."""
    src = inspect.getsource(omlp)
    assert src.count(old) == 1, f"mutation site not unique: {old!r}"
    mod = types.ModuleType("oracle._mlp_mutant")
    mod.__package__ = "oracle"
    exec(compile(src.replace(old, new), "<oracle/mlp.py mutant>", "exec"), mod.__dict__)
    return mod


MUTANTS = {
    "gate_up_swapped": ("g = bf(gu[:, :N].float()", "g = bf(gu[:, N:].float()"),
    "dg_du_swapped_in_dx_operand": ("mx.quant(torch.cat([dg, du], 1))", "mx.quant(torch.cat([du, dg], 1))"),
    "s_d_dropped_from_dB_d": ("dB_d = (dB_d.float() * s_d).to(BF16)", "dB_d = dB_d"),
    "dxa_scaled_after_rounding": ("dxa_g = dxa_g * s_g", "dxa_g = bf(dxa_g) * s_g"),
    "wrong_swiglu_derivative": ("(g * (1.0 - sig) + 1.0)", "(1.0 - sig)"),
    "down_lora_B_dropped": ("y = (y0.float() + s_d * (xsd.float() @ bd.float().t())).to(BF16)", "y = y0"),
    "dxa_g_takes_B_u": ("dxa_g = dg.float() @ bg.float()", "dxa_g = dg.float() @ bu.float()"),
    "xs_down_takes_B_d_rows": ("xS = h.float() @ ad.float().t()", "xS = h.float() @ ad.float().flip(0).t()"),
    "dB_d_rounded_once": ("dB_d = (dy2.float().t() @ bf(xS)).to(BF16)", "dB_d = dy2.float().t() @ bf(xS)"),
    "dx_lora_term_dropped": ("dx = (dx0.float() + dxa.float() @ S.float()).to(BF16)", "dx = dx0"),
    "wt_transposed_weight": ("wt, wts = mx.quant_t(Wgu)", "wt, wts = mx.quant(Wgu.t().contiguous().t().contiguous())"),
}


# The checks that must reject each mutant.  Every mutant but the pure rounding-point ones is rejected by a
# check that uses no oracle code (the float64 composition, autograd or central differences).
_F64_CHECKS = {"check_forward", "check_autograd", "check_finite_differences"}
EXPECT = {
    "gate_up_swapped": _F64_CHECKS,
    "dg_du_swapped_in_dx_operand": {"check_autograd", "check_finite_differences", "check_rounding_points"},
    "s_d_dropped_from_dB_d": {"check_autograd", "check_finite_differences", "check_rounding_points",
                              "check_zero_scalings"},
    "dxa_scaled_after_rounding": {"check_rounding_points"},
    "wrong_swiglu_derivative": {"check_autograd", "check_finite_differences", "check_rounding_points"},
    "down_lora_B_dropped": {"check_forward"},
    "dxa_g_takes_B_u": {"check_autograd", "check_finite_differences", "check_rounding_points"},
    "xs_down_takes_B_d_rows": {"check_autograd", "check_finite_differences", "check_rounding_points"},
    "dB_d_rounded_once": {"check_rounding_points"},
    "dx_lora_term_dropped": {"check_autograd", "check_rounding_points"},  # small next to dx: not FD-visible
    "wt_transposed_weight": {"check_weights", "check_autograd", "check_finite_differences"},
}


def rejections(mod, c):
    out = set()
    for chk in CHECKS:
        try:
            chk(c, mod)
        except Exception:  # an assertion, or a shape / index error
            out.add(chk.__name__)
    return out


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_checks_reject_mutant(name, case):
    """Every planted mistake is rejected by the checks listed for it (at least)."""
    got = rejections(_mutant(*MUTANTS[name]), case)
    assert EXPECT[name] <= got, (name, sorted(got))


def test_every_mutant_has_expectations():
    assert set(EXPECT) == set(MUTANTS)
