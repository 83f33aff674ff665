"""GPU parity of the fused MXFP8 SwiGLU MLP (fused_mlp.mlp / _MLP on libmxfp8_mlp.so) against the CPU oracle.

Bars (north star):
  - quantized codes and scales bit-exact: x and dy directly; h and dg|du given the same bf16 values (the GPU's
    own h / dg / du are quantized by the oracle and compared byte for byte);
  - h, dg, du themselves within one bf16 ulp of the oracle on identical inputs (they differ only by fp32
    summation order of the rank-r products and exp/division ulps);
  - GEMM/MLP outputs and LoRA gradients: max|Δ| / max|ref| <= 2e-2 against the oracle's dequantize-then-
    matmul path (TOL below)."""
import numpy as np
import pytest
import torch

import fused_linear
import fused_mlp
import mxfp8
import workloads
from oracle import mlp as omlp
from oracle import mx

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _rel(got, ref):
    got, ref = got.float().cpu(), ref.float().cpu()
    return ((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()


def _ulp_ok(got, ref):
    """bf16 tensors computed from identical inputs: g and u can land one ulp apart when the fp32 rank-r LoRA sum
    (different summation order) sits on a bf16 rounding boundary, and silu / its derivative amplify that into
    a few ulps of h, dg, du.  Bar: at most 1e-4 of the elements differ by more than one bf16 ulp and none by
    more than 2^-4 relative (plus 2^-20 of max|ref| absolute).  Returns the fraction of inexact elements."""
    got, ref = got.float().cpu(), ref.float().cpu()
    d = (got - ref).abs()
    mag = torch.maximum(got.abs(), ref.abs())
    ulp = torch.exp2(torch.floor(torch.log2(mag.clamp_min(2.0 ** -126))) - 7)
    beyond = (d > ulp).float().mean().item()
    assert beyond <= 1e-4, beyond
    assert bool((d <= 2.0 ** -4 * mag + 2.0 ** -20 * ref.abs().max()).all()), d.max().item()
    return (got != ref).float().mean().item()


def _oracle_all(inp, backward=True):
    W = omlp.prepare_weights(inp["Wg"], inp["Wu"], inp["Wd"])
    S, bg, bu, ad, bd = omlp.lora_cast(inp["Ag"], inp["Bg"], inp["Au"], inp["Bu"], inp["Ad"], inp["Bd"])
    s = inp["s"]
    f = omlp.forward(inp["x"], W, S, bg, bu, ad, bd, s, s, s)
    b = omlp.backward(inp["x"], f["xs"], f["gu"], W, S, bg, bu, ad, bd, s, s, s, inp["dy"]) if backward else None
    return W, (S, bg, bu, ad, bd), f, b


def _run_model(cfg, T, gpu, backward=True, need_out=True):
    model, inps = workloads.build_model(cfg, T=T, device=gpu)
    mxfp8.enable_mxfp8(model)
    fused_linear.new_step()
    inp = inps[0]
    mod = model.layers[0].mlp
    x = inp["x"].to(gpu).requires_grad_(backward)
    y = fused_mlp.mlp(mod, x, need_out)
    assert y is not None
    out = dict(y=y.detach())
    if backward:
        y.backward(inp["dy"].to(gpu))
        out.update(dx=x.grad, dA_g=mod.gate_proj.lora_A["default"].weight.grad,
                   dB_g=mod.gate_proj.lora_B["default"].weight.grad,
                   dA_u=mod.up_proj.lora_A["default"].weight.grad, dB_u=mod.up_proj.lora_B["default"].weight.grad,
                   dA_d=mod.down_proj.lora_A["default"].weight.grad,
                   dB_d=mod.down_proj.lora_B["default"].weight.grad)
    return model, inp, out


def _check_e2e(out, ref_f, ref_b):
    errs = {"y": _rel(out["y"], ref_f["y"])}
    if ref_b is not None:
        for k in ("dx", "dA_g", "dB_g", "dA_u", "dB_u", "dA_d", "dB_d"):
            errs[k] = _rel(out[k], ref_b[k])
    print(" ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    bad = {k: v for k, v in errs.items() if not v <= TOL}
    assert not bad, bad


@pytest.mark.parametrize("cfg,T", [(1, None), (2, 1024), (2, 300), (3, 512), (5, 1024)])
def test_mlp_end_to_end(cfg, T, gpu):
    bwd = workloads.CONFIGS[cfg]["backward"]
    print(f"config {cfg} T={T}", flush=True)
    _, inp, out = _run_model(cfg, T, gpu, backward=bwd)
    _, _, f, b = _oracle_all(inp, backward=bwd)
    _check_e2e(out, f, b)


def test_mlp_end_to_end_config2_full(gpu):
    _, inp, out = _run_model(2, None, gpu)
    _, _, f, b = _oracle_all(inp)
    _check_e2e(out, f, b)


_EXTRA = {
    # rank 32 (the reference's other accepted rank): the fused kernels' R = 32 variants and the 2r = 64 products
    61: dict(name="r32", T=1000, K=1024, N=3584, r=32, alpha=64, backward=True, layers=1),
    # d_model and d_ffn odd multiples of 128 (the reference's gate is d_ffn % 128 == 0), at both ranks
    62: dict(name="odd128", T=700, K=384, N=640, r=16, alpha=32, backward=True, layers=1),
    63: dict(name="odd128_r32", T=333, K=384, N=640, r=32, alpha=64, backward=True, layers=1),
}


@pytest.mark.parametrize("cfg", sorted(_EXTRA))
def test_mlp_end_to_end_other_shapes(cfg, gpu, monkeypatch):
    monkeypatch.setitem(workloads.CONFIGS, cfg, _EXTRA[cfg])
    print(f"shape {_EXTRA[cfg]}", flush=True)
    _, inp, out = _run_model(cfg, None, gpu)
    _, _, f, b = _oracle_all(inp)
    _check_e2e(out, f, b)


@pytest.mark.parametrize("cfg", [3, 5])
def test_mlp_end_to_end_full_size(cfg, gpu):
    # the headline shape (T=10752, d_model 2048, d_ffn 6144) and its outlier variant at full size: the GPU path
    # against the oracle (about 20-30 s of CPU and 6 GB of host memory each)
    print(f"config {cfg} full size", flush=True)
    _, inp, out = _run_model(cfg, None, gpu)
    _, _, f, b = _oracle_all(inp)
    _check_e2e(out, f, b)


def _kernel_inputs(cfg, T, gpu):
    inp = workloads.make_inputs(cfg, T=T)
    W, (S, bg, bu, ad, bd), f, b = _oracle_all(inp)
    g = lambda t: t.to(gpu).contiguous()  # noqa: E731
    return inp, W, (S, bg, bu, ad, bd), f, b, g


@pytest.mark.parametrize("cfg,T", [(2, 512), (3, 300), (5, 1024)])
def test_fwd_kernel_elementwise_and_codes(cfg, T, gpu):
    inp, W, (S, bg, bu, ad, bd), f, b, g = _kernel_inputs(cfg, T, gpu)
    N, s = inp["N"], inp["s"]
    h = torch.empty(T, N, dtype=torch.bfloat16, device=gpu)
    qh, sh, xsd = fused_mlp.mlp_fwd(g(f["gu"]), g(f["xs"]), g(bg), g(bu), g(ad), s, s, True, h_out=h)
    frac = _ulp_ok(h, f["h"])
    print(f"h: {frac:.2e} of elements differ by one ulp", flush=True)
    assert frac < 1e-3
    # codes and scales of h bit-exact given the same bf16 h
    qr, sr = mx.quant(h.cpu())
    assert torch.equal(qh.view(torch.uint8).cpu(), qr) and torch.equal(sh.view(torch.uint8).cpu(), sr)
    # xS_down = bf16(h · adᵀ) from the GPU's own h
    ref = (h.cpu().double() @ ad.double().t())
    assert _rel(xsd, ref) <= 1e-2
    # the MX-tiled output (the GEMM operand layout of the fused path) holds the same codes
    qt, st, xsd_t = fused_mlp.mlp_fwd(g(f["gu"]), g(f["xs"]), g(bg), g(bu), g(ad), s, s, True, tiled=True)
    assert torch.equal(st, sh) and torch.equal(xsd_t, xsd)
    assert np.array_equal(mx.from_tiled(qt.view(torch.uint8).cpu().numpy().reshape(-1), T, N), qr.numpy())
    # gu in the fused-tile layout (what the fused path's GEMM writes): bit-identical results
    gu_ft = torch.from_numpy(mx.to_ft(f["gu"].view(torch.uint16).numpy()).view(np.int16)).view(torch.bfloat16)
    qf, sf, xsd_f = fused_mlp.mlp_fwd(g(gu_ft.view(-1, 2 * N)), g(f["xs"]), g(bg), g(bu), g(ad), s, s, True,
                                      tiled=True, gu_ft=True)
    live = lambda qq, C: mx.from_tiled(qq.view(torch.uint8).cpu().numpy().reshape(-1), T, C)  # noqa: E731
    assert np.array_equal(live(qf, N), live(qt, N)) and torch.equal(sf, st) and torch.equal(xsd_f, xsd)


@pytest.mark.parametrize("cfg,T", [(2, 512), (3, 300), (5, 1024)])
def test_bwd_kernel_elementwise_and_codes(cfg, T, gpu):
    inp, W, (S, bg, bu, ad, bd), f, b, g = _kernel_inputs(cfg, T, gpu)
    N, R, s = inp["N"], inp["r"], inp["s"]
    dgu = torch.empty(T, 2 * N, dtype=torch.bfloat16, device=gpu)
    q, sc, dxa, dbg, dbu, dad = fused_mlp.mlp_bwd(g(f["gu"]), g(f["xs"]), g(b["dhm"]), g(b["dxd"]), g(bg), g(bu),
                                                  g(ad), s, s, True, dgu_out=dgu)
    fg = _ulp_ok(dgu[:, :N], b["dg"])
    fu = _ulp_ok(dgu[:, N:], b["du"])
    print(f"dg: {fg:.2e}, du: {fu:.2e} of elements differ by one ulp", flush=True)
    assert fg < 1e-2 and fu < 1e-2
    qr, sr = mx.quant(dgu.cpu())
    assert torch.equal(q.view(torch.uint8).cpu(), qr) and torch.equal(sc.view(torch.uint8).cpu(), sr)
    qt, sct = fused_mlp.mlp_bwd(g(f["gu"]), g(f["xs"]), g(b["dhm"]), g(b["dxd"]), g(bg), g(bu), g(ad), s, s, True,
                                tiled=True)[:2]
    assert torch.equal(sct, sc)
    assert np.array_equal(mx.from_tiled(qt.view(torch.uint8).cpu().numpy().reshape(-1), T, 2 * N), qr.numpy())
    # gu and dhm in the fused-tile layout: bit-identical results
    ft = lambda t: torch.from_numpy(mx.to_ft(t.view(torch.uint16).numpy()).view(np.int16)).view(  # noqa: E731
        torch.bfloat16).view(-1, t.shape[1])
    outs_rm = fused_mlp.mlp_bwd(g(f["gu"]), g(f["xs"]), g(b["dhm"]), g(b["dxd"]), g(bg), g(bu), g(ad), s, s, True,
                                tiled=True)
    outs_ft = fused_mlp.mlp_bwd(g(ft(f["gu"])), g(f["xs"]), g(ft(b["dhm"])), g(b["dxd"]), g(bg), g(bu), g(ad), s, s,
                                True, tiled=True, gu_ft=True)
    # (the tiled code buffer's padding rows past T are never written: compare its live rows)
    assert np.array_equal(mx.from_tiled(outs_rm[0].view(torch.uint8).cpu().numpy().reshape(-1), T, 2 * N),
                          mx.from_tiled(outs_ft[0].view(torch.uint8).cpu().numpy().reshape(-1), T, 2 * N))
    for a_, b_ in zip(outs_rm[1:], outs_ft[1:]):
        assert torch.equal(a_, b_)
    # partial-sum products from the GPU's own dg / du and the oracle's h, in float64
    dg64, du64 = dgu[:, :N].cpu().double(), dgu[:, N:].cpu().double()
    h64 = b["h"].double()
    xs64, dxd64 = f["xs"].double(), b["dxd"].double()
    assert _rel(dxa[:, :R], dg64 @ bg.double()) <= 1e-2
    assert _rel(dxa[:, R:2 * R], du64 @ bu.double()) <= 1e-2
    assert _rel(dxa[:, 2 * R:], h64 @ ad.double().t()) <= 1e-2
    assert _rel(dbg, dg64.t() @ xs64[:, :R]) <= 1e-2
    assert _rel(dbu, du64.t() @ xs64[:, R:]) <= 1e-2
    assert _rel(dad, (h64.t() @ dxd64).t()) <= 1e-2
    # and against the oracle's own unscaled partials
    assert _rel(dxa, b["dxa_raw"]) <= TOL and _rel(dbg, b["dBg_raw"]) <= TOL and _rel(dad, b["dAd"]) <= TOL


@pytest.mark.parametrize("wide,sb,cg", [(True, 128, 512), (True, 384, 1792), (False, 256, 256), (False, 128, 896)])
def test_bwd_kernel_grids_with_several_column_passes(wide, sb, cg, gpu, monkeypatch):
    """The backward kernel with grids whose workgroups walk several column passes (CG > 128 · waves / 4) and
    super-blocks of several sizes, T = 300 (rows past T in the last super-block): its staged small operands
    restart at each pass.  The MX codes and scales of dg | du and the dxa partials' column partition do not depend
    on the grid, so codes, scales and (8-wave, one partial per 256 columns either way) dxa are bit-identical to
    the default grid's; the dB / dA_d sums group the rows by super-block, so they agree to fp32 rounding."""
    inp, W, (S, bg, bu, ad, bd), f, b, g = _kernel_inputs(2, 300, gpu)
    s = inp["s"]
    args = (g(f["gu"]), g(f["xs"]), g(b["dhm"]), g(b["dxd"]), g(bg), g(bu), g(ad), s, s, True)
    monkeypatch.setattr(fused_mlp, "WIDE_BWD", [wide])
    ref = fused_mlp.mlp_bwd(*args, tiled=True)
    assert fused_mlp.LAST["bwd"]["wide"] == wide
    monkeypatch.setattr(fused_mlp, "_bwd_grid", lambda T, N, R, wide=False: (sb, cg))
    out = fused_mlp.mlp_bwd(*args, tiled=True)
    assert (fused_mlp.LAST["bwd"]["SB"], fused_mlp.LAST["bwd"]["CG"]) == (sb, cg)
    T, N = 300, inp["N"]
    assert np.array_equal(mx.from_tiled(out[0].view(torch.uint8).cpu().numpy().reshape(-1), T, 2 * N),
                          mx.from_tiled(ref[0].view(torch.uint8).cpu().numpy().reshape(-1), T, 2 * N))
    assert torch.equal(out[1], ref[1])
    assert torch.equal(out[2], ref[2])
    for a_, b_ in zip(out[3:], ref[3:]):
        assert _rel(a_, b_.cpu().double()) <= 1e-6


def test_need_out_false_saves_same_and_backward_matches(gpu):
    # checkpoint recompute: need_out=False leaves the saved set and therefore every gradient unchanged
    _, _, out1 = _run_model(2, 384, gpu, need_out=True)
    _, _, out2 = _run_model(2, 384, gpu, need_out=False)
    for k in ("dx", "dA_g", "dB_g", "dA_u", "dB_u", "dA_d", "dB_d"):
        assert torch.equal(out1[k], out2[k]), k


def test_deterministic(gpu):
    _, _, o1 = _run_model(3, 640, gpu)
    _, _, o2 = _run_model(3, 640, gpu)
    for k, v in o1.items():
        assert torch.equal(v, o2[k]), k


def test_lora_b_zero_gives_zero_a_grads(gpu):
    # with every LoRA B = 0: dA_g = dA_u = dA_d = 0 exactly, and y equals the plain MX SwiGLU of the oracle
    model, inps = workloads.build_model(2, T=256, device=gpu)
    mod = model.layers[0].mlp
    with torch.no_grad():
        for name in ("gate_proj", "up_proj", "down_proj"):
            getattr(mod, name).lora_B["default"].weight.zero_()
    mxfp8.enable_mxfp8(model)
    fused_linear.new_step()
    inp = inps[0]
    x = inp["x"].to(gpu).requires_grad_(True)
    y = fused_mlp.mlp(mod, x)
    y.backward(inp["dy"].to(gpu))
    for name in ("gate_proj", "up_proj", "down_proj"):
        assert int(torch.count_nonzero(getattr(mod, name).lora_A["default"].weight.grad)) == 0
    zero = {k: torch.zeros_like(inp[k]) for k in ("Bg", "Bu", "Bd")}
    _, _, f, _ = _oracle_all({**inp, **zero}, backward=False)
    assert _rel(y, f["y"]) <= TOL


def test_mlp_gating_returns_none(gpu):
    model, inps = workloads.build_model(1, T=64, device=gpu)
    mod = model.layers[0].mlp
    x = inps[0]["x"].to(gpu)
    assert fused_mlp.mlp(mod, x) is None  # weights not prepared by enable_mxfp8
    mxfp8.enable_mxfp8(model)
    assert fused_mlp.mlp(mod, x.float()) is None  # not bf16
    assert fused_mlp.mlp(mod, inps[0]["x"]) is None  # CPU tensor
    fused_mlp.ENABLED[0] = False
    try:
        assert fused_mlp.mlp(mod, x) is None
    finally:
        fused_mlp.ENABLED[0] = True
    assert fused_mlp.mlp(mod, x) is not None


def test_config4_one_conversation(gpu):
    # one packed conversation of the training-step shape: 8896 % 128 = 64 leaves half of the last scale tile
    # padded (its rows must encode as scale 0)
    _, inp, out = _run_model(4, 8896, gpu)
    _, _, f, b = _oracle_all(inp)
    _check_e2e(out, f, b)


def test_config4_two_layer_stack(gpu):
    # a stack feeds layer 1 the output of layer 0 and chains the backward through it; each layer is checked
    # against the oracle on the GPU's own tensors at the layer boundary (y0 forward, dL/dy0 backward), since
    # two independently quantized chains drift apart by more than one layer's tolerance
    T = 384
    model, inps = workloads.build_model(4, T=T, layers=2, device=gpu)
    mxfp8.enable_mxfp8(model)
    fused_linear.new_step()
    m0, m1 = model.layers[0].mlp, model.layers[1].mlp
    x = inps[0]["x"].to(gpu).requires_grad_(True)
    y0 = fused_mlp.mlp(m0, x)
    y0.retain_grad()
    y1 = fused_mlp.mlp(m1, y0)
    y1.backward(inps[0]["dy"].to(gpu))
    ref1 = {**inps[1], "x": y0.detach().cpu(), "dy": inps[0]["dy"]}
    _, _, f1, b1 = _oracle_all(ref1)
    ref0 = {**inps[0], "dy": y0.grad.cpu()}
    _, _, f0, b0 = _oracle_all(ref0)
    errs = {"y0": _rel(y0, f0["y"]), "y1": _rel(y1, f1["y"]), "dy0": _rel(y0.grad, b1["dx"]),
            "dx": _rel(x.grad, b0["dx"])}
    for i, (m, b) in enumerate(((m0, b0), (m1, b1))):
        for k, (name, ab) in {"dA_g": ("gate_proj", "A"), "dB_g": ("gate_proj", "B"), "dA_d": ("down_proj", "A"),
                              "dB_d": ("down_proj", "B")}.items():
            errs[f"{k}{i}"] = _rel(getattr(getattr(m, name), f"lora_{ab}")["default"].weight.grad, b[k])
    print(" ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert all(v <= TOL for v in errs.values()), errs
