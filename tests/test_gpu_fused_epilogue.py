"""GPU parity of the GEMMs with the SwiGLU epilogues against the separate paths they replace, which the oracle
pins (tests/test_gpu_mlp.py).
  - forward: the gate|up GEMM with the SwiGLU forward in its epilogue (mxfp8.swiglu_gemm -> mxfp8_gemm_swiglu_fwd)
    against the FT-output MX GEMM, then the fused forward kernel mlp_fwd: on identical operands gu, the MX codes
    of h and their scales are bit-identical (same products, same epilogue arithmetic); xS_down is added over
    other partial groupings (one partial per 128-column tile instead of per column group), so it is within one
    bf16 step;
  - backward: the dgrad GEMM of h with the SwiGLU backward in its epilogue (mxfp8.swiglu_bwd_gemm ->
    mxfp8_gemm_swiglu_bwd) against the FT-output MX GEMM dhm, then the fused backward kernel mlp_bwd (below)."""
import pytest
import torch

import fused_linear
import fused_mlp
import mxfp8
import workloads
from oracle import mx

pytestmark = pytest.mark.gpu


def _ft_rows(t, T, C):
    return torch.from_numpy(mx.from_ft(t.view(torch.int16).cpu().reshape(-1).numpy(), T, C))


def _tiled_rows(q, T, C):
    return torch.from_numpy(mx.from_tiled(q.view(torch.uint8).cpu().reshape(-1).numpy(), T, C))


@pytest.mark.parametrize("cfg,T", [(3, 300), (2, 1000), (5, 1024), (61, 500), (62, 333), (3, None)])
def test_fused_forward_matches_separate_path(cfg, T, gpu, monkeypatch):
    extra = {61: dict(name="r32", T=1000, K=1024, N=3584, r=32, alpha=64, backward=True, layers=1),
             62: dict(name="odd128", T=700, K=384, N=640, r=16, alpha=32, backward=True, layers=1)}
    if cfg in extra:
        monkeypatch.setitem(workloads.CONFIGS, cfg, extra[cfg])
    model, inps = workloads.build_model(cfg, T=T, device=gpu)
    mxfp8.enable_mxfp8(model)
    fused_linear.new_step()
    inp, mod = inps[0], model.layers[0].mlp
    T, N, s = inp["T"], inp["N"], inp["s"]
    print(f"config {cfg} T={T} N={N} r={inp['r']}", flush=True)
    hold = mod.gate_proj.base_layer._mx_gu[0]
    g = lambda m: m.lora_A["default"].weight, lambda m: m.lora_B["default"].weight  # noqa: E731
    lw = fused_mlp._prep(g[0](mod.gate_proj), g[1](mod.gate_proj), g[0](mod.up_proj), g[1](mod.up_proj),
                         g[0](mod.down_proj), g[1](mod.down_proj), torch.bfloat16)
    x = inp["x"].to(gpu)
    if 2 * inp["r"] <= 32:
        q, sc, xs, _ = mxfp8.mx_quant_lora(x, lw.S, out_t=False)
    else:
        import _native
        xs = torch.empty((T, 2 * inp["r"]), dtype=torch.bfloat16, device=gpu)
        _native.lora_nt(x, lw.S, xs)
        q, sc = mxfp8.mx_quant_tiled(x)
    gu0 = mxfp8.mx_mm(q, sc, hold.w_tl, hold.ws, layout=fused_mlp._LAYOUT_FT, m=T)
    qh0, sh0, xsd0 = fused_mlp.mlp_fwd(gu0, xs, lw.bg, lw.bu, lw.ad, s, s, True, tiled=True, gu_ft=True)
    gu1, qh1, sh1, part = mxfp8.swiglu_gemm(q, sc, hold, xs, lw.bg, lw.bu, lw.ad, s, s, T)
    xsd1 = part.sum(0).to(torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(_ft_rows(gu1, T, 2 * N), _ft_rows(gu0, T, 2 * N)), "gu"
    assert torch.equal(_tiled_rows(qh1, T, N), _tiled_rows(qh0, T, N)), "codes of h"
    assert torch.equal(sh1.view(torch.uint8), sh0.view(torch.uint8)), "scales of h (padded rows 0)"
    a, b = xsd1.float().cpu(), xsd0.float().cpu()
    d = (a - b).abs()
    ulp = torch.exp2(torch.floor(torch.log2(torch.maximum(a.abs(), b.abs()).clamp_min(2.0 ** -126))) - 7)
    assert bool((d <= ulp).all()), d.max().item()


@pytest.mark.parametrize("cfg,T", [(3, 300), (2, 1000), (5, 1024), (62, 333), (2, 1100), (3, None)])
def test_fused_backward_matches_separate_path(cfg, T, gpu, monkeypatch):
    """The dgrad GEMM of h with the SwiGLU backward in its epilogue (mxfp8.swiglu_bwd_gemm ->
    mxfp8_gemm_swiglu_bwd) against the separate path (the FT-output MX GEMM dhm = MX(dy)·W_down, then the
    fused backward kernel mlp_bwd), on identical operands: the MX codes and scales of dg | du and the per-tile
    dxa | dxa_u | xS_down partials are bit-identical (same products, same order of the column sums); the dB_g,
    dB_u and dA_d partials group the rows by 256-row tiles instead of the kernel's super-blocks, so their sums
    agree to fp32 rounding.  T = 300, 333, 1100 leave partial 256-row tiles, with blocks past the padded rows."""
    extra = {62: dict(name="odd128", T=700, K=384, N=640, r=16, alpha=32, backward=True, layers=1)}
    if cfg in extra:
        monkeypatch.setitem(workloads.CONFIGS, cfg, extra[cfg])
    model, inps = workloads.build_model(cfg, T=T, device=gpu)
    mxfp8.enable_mxfp8(model)
    fused_linear.new_step()
    inp, mod = inps[0], model.layers[0].mlp
    T, N, s = inp["T"], inp["N"], inp["s"]
    print(f"config {cfg} T={T} N={N} r={inp['r']}", flush=True)
    hold, down = mod.gate_proj.base_layer._mx_gu[0], mod.down_proj.base_layer
    g = lambda m: m.lora_A["default"].weight, lambda m: m.lora_B["default"].weight  # noqa: E731
    lw = fused_mlp._prep(g[0](mod.gate_proj), g[1](mod.gate_proj), g[0](mod.up_proj), g[1](mod.up_proj),
                         g[0](mod.down_proj), g[1](mod.down_proj), torch.bfloat16)
    x, dy = inp["x"].to(gpu), inp["dy"].to(gpu)
    q, sc, xs, _ = mxfp8.mx_quant_lora(x, lw.S, out_t=False)
    gu, _, _, _ = mxfp8.swiglu_gemm(q, sc, hold, xs, lw.bg, lw.bu, lw.ad, s, s, T)
    xsT = fused_mlp._transposed_padded(xs, -(-T // 128) * 128)
    qd, sd, dxd, dxdT = mxfp8.mx_quant_lora(dy, lw.bdT, scale=s)
    dhm = mxfp8.mx_mm(qd, sd, down._mx_wt_tl, down._mx_wts, layout=fused_mlp._LAYOUT_FT, m=T)
    q0, s0, p0 = fused_mlp._bwd_launch(gu, xs, xsT, dhm, dxd, dxdT, lw.bg, lw.bu, lw.bgT, lw.buT, lw.ad, lw.adT, s, s,
                                       True, None, True, gu_ft=True, wide=False)
    q1, s1, p1 = mxfp8.swiglu_bwd_gemm(qd, sd, down, gu, xs, xsT, dxd, dxdT, lw.bg, lw.bgT, lw.bu, lw.buT, lw.ad,
                                       lw.adT, s, s, T)
    torch.cuda.synchronize()
    assert torch.equal(_tiled_rows(q1, T, 2 * N), _tiled_rows(q0, T, 2 * N)), "codes of dg | du"
    assert torch.equal(s1.view(torch.uint8), s0.view(torch.uint8)), "scales of dg | du (padded rows 0)"
    assert p1[0].shape == p0[0].shape and torch.equal(p1[0], p0[0]), "dxa | dxa_u | xS_down partials"
    assert p1[1].shape[0] == -(-T // 256)
    for k, name in ((1, "dB_g"), (2, "dB_u"), (3, "dA_d")):
        a, b = p1[k].double().sum(0).cpu(), p0[k].double().sum(0).cpu()
        err = ((a - b).abs().max() / b.abs().max()).item()
        assert err <= 1e-5, (name, err)


def test_fused_backward_autograd_matches_separate_path(gpu):
    """The whole _MLP step with both epilogues fused and with neither (FUSED_EPILOGUE): y within a bf16 step (the
    forward's xS_down partials are grouped differently); dx, dA_g, dA_u, dB_d bit-identical (the backward
    recomputes h and xS_down from gu); dB_g, dB_u, dA_d to fp32 rounding of their partial sums."""
    out = []
    for fused in (False, True):
        # the split path with one dxa partial per 128 columns, the grouping of the fused epilogue
        fused_mlp.FUSED_EPILOGUE[0] = fused_mlp.FUSED_BWD_EPILOGUE[0] = fused
        fused_mlp.WIDE_BWD[0] = False
        try:
            model, inps = workloads.build_model(3, T=2000, device=gpu)
            mxfp8.enable_mxfp8(model)
            fused_linear.new_step()
            mod = model.layers[0].mlp
            x = inps[0]["x"].to(gpu).requires_grad_(True)
            y = fused_mlp.mlp(mod, x)
            y.backward(inps[0]["dy"].to(gpu))
            torch.cuda.synchronize()
            gr = {n: p.grad.detach().clone() for n, p in mod.named_parameters() if p.requires_grad}
            out.append((y.detach(), x.grad.detach(), gr))
        finally:
            fused_mlp.FUSED_EPILOGUE[0], fused_mlp.FUSED_BWD_EPILOGUE[0], fused_mlp.WIDE_BWD[0] = True, False, True
    (y0, dx0, g0), (y1, dx1, g1) = out
    assert torch.equal(dx0, dx1)
    a, b = y1.float(), y0.float()
    assert bool(((a - b).abs() <= b.abs() * 2.0 ** -7 + 1e-3 * b.abs().max()).all())
    for n in g0:
        if "gate_proj.lora_A" in n or "up_proj.lora_A" in n or "down_proj.lora_B" in n:
            assert torch.equal(g0[n], g1[n]), n
        else:
            err = ((g1[n] - g0[n]).abs().max() / g0[n].abs().max()).item()
            assert err <= 1e-5, (n, err)


@pytest.mark.parametrize("cfg,T", [(3, 1100), (5, 600)])
def test_wide_backward_matches_narrow(cfg, T, gpu):
    """The 8-wave backward workgroups (one dxa partial per 256 columns, two quads summed in LDS) against the 4-wave
    ones (one per 128 columns, the pairs added by the finish): MX codes and scales of dg | du bit-identical, each
    wide dxa partial equal to the sum of its two narrow ones and the dB / dA_d sums equal, to fp32 rounding."""
    model, inps = workloads.build_model(cfg, T=T, device=gpu)
    mxfp8.enable_mxfp8(model)
    fused_linear.new_step()
    inp, mod = inps[0], model.layers[0].mlp
    T, N, s = inp["T"], inp["N"], inp["s"]
    hold, down = mod.gate_proj.base_layer._mx_gu[0], mod.down_proj.base_layer
    g = lambda m: m.lora_A["default"].weight, lambda m: m.lora_B["default"].weight  # noqa: E731
    lw = fused_mlp._prep(g[0](mod.gate_proj), g[1](mod.gate_proj), g[0](mod.up_proj), g[1](mod.up_proj),
                         g[0](mod.down_proj), g[1](mod.down_proj), torch.bfloat16)
    x, dy = inp["x"].to(gpu), inp["dy"].to(gpu)
    q, sc, xs, _ = mxfp8.mx_quant_lora(x, lw.S, out_t=False)
    gu, _, _, _ = mxfp8.swiglu_gemm(q, sc, hold, xs, lw.bg, lw.bu, lw.ad, s, s, T)
    xsT = fused_mlp._transposed_padded(xs, -(-T // 128) * 128)
    qd, sd, dxd, dxdT = mxfp8.mx_quant_lora(dy, lw.bdT, scale=s)
    dhm = mxfp8.mx_mm(qd, sd, down._mx_wt_tl, down._mx_wts, layout=fused_mlp._LAYOUT_FT, m=T)
    args = (gu, xs, xsT, dhm, dxd, dxdT, lw.bg, lw.bu, lw.bgT, lw.buT, lw.ad, lw.adT, s, s, True, None, True)
    q0, s0, p0 = fused_mlp._bwd_launch(*args, gu_ft=True, wide=False)
    q1, s1, p1 = fused_mlp._bwd_launch(*args, gu_ft=True, wide=True)
    torch.cuda.synchronize()
    assert fused_mlp.LAST["bwd"]["wide"] and p1[0].shape[0] * 2 == p0[0].shape[0]
    assert torch.equal(_tiled_rows(q1, T, 2 * N), _tiled_rows(q0, T, 2 * N)), "codes of dg | du"
    assert torch.equal(s1.view(torch.uint8), s0.view(torch.uint8)), "scales of dg | du"
    pairs = p0[0].double().view(-1, 2, T, p0[0].shape[2]).sum(1)
    err = ((p1[0].double() - pairs).abs().max() / pairs.abs().max()).item()
    assert err <= 1e-6, err
    for k, name in ((1, "dB_g"), (2, "dB_u"), (3, "dA_d")):
        a, b = p1[k].double().sum(0), p0[k].double().sum(0)
        err = ((a - b).abs().max() / b.abs().max()).item()
        assert err <= 1e-5, (name, err)
